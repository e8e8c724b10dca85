"""ctypes access to the checkers under oracle/ (the CPU restatement and, when built, the
reference's own expert path). Test infrastructure: imported by tests/ and bench.py's
cpu_baseline leg only."""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_LIB = os.path.join(ROOT, "oracle", "lib", "libg53_oracle.so")
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libglm53f_ref.so")


class OrExpert(C.Structure):
    _fields_ = [("gw", C.c_void_p), ("uw", C.c_void_p), ("dw", C.c_void_p),
                ("gs", C.c_void_p), ("us", C.c_void_p), ("ds", C.c_void_p)]


_or = None
_ref = None


def oracle():
    global _or
    if _or is None:
        L = C.CDLL(ORACLE_LIB)
        L.or_e4m3f.restype = C.c_float
        L.or_e4m3f.argtypes = [C.c_uint8]
        L.or_mm_f8.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                               C.c_int, C.c_int]
        L.or_swiglu.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_float]
        L.or_router.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                C.c_int, C.c_int, C.c_float]
        L.or_route_topn.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int]
        L.or_moe.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                             C.c_int, C.c_float, C.c_float, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                             C.c_void_p, C.c_void_p]
        L.or_expf_mismatches.restype = C.c_long
        L.or_expf_mismatches.argtypes = [C.c_void_p, C.c_uint32, C.c_long, C.POINTER(C.c_long)]
        L.or_expf.argtypes = [C.c_void_p, C.c_void_p, C.c_long]
        L.or_mm_i4.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]
        L.or_i4_from_f8.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                    C.c_int]
        L.or_moe_i4.argtypes = L.or_moe.argtypes
        _or = L
    return _or


def have_ref():
    return os.path.exists(REF_LIB)


def ref():
    global _ref
    if _ref is None:
        L = C.CDLL(REF_LIB)
        L.ref_moe.restype = C.c_long
        L.ref_moe.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                              C.c_int, C.c_int, C.c_float, C.c_float, C.c_void_p, C.c_void_p, C.c_void_p,
                              C.c_void_p]
        L.ref_router.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int,
                                 C.c_float, C.c_void_p, C.c_void_p]
        L.ref_mm.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                             C.c_int, C.c_int]
        L.ref_swiglu.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_float]
        if hasattr(L, "ref_cache_trace"):
            L.ref_cache_trace.restype = C.c_int
            L.ref_cache_trace.argtypes = [C.c_char_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int,
                                          C.c_void_p, C.c_void_p, C.c_void_p]
        L.ref_moe_i4.restype = C.c_long
        L.ref_moe_i4.argtypes = L.ref_moe.argtypes
        L.ref_mm_i4.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int]
        L.ref_i4_from_f8.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                     C.c_int]
        L.ref_e4m3f.restype = C.c_float
        L.ref_e4m3f.argtypes = [C.c_uint8]
        if hasattr(L, "ref_moe_proto"):
            L.ref_moe_proto.restype = C.c_int
            L.ref_moe_proto.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                        C.c_int, C.c_int, C.c_float, C.c_float, C.c_void_p, C.c_void_p, C.c_void_p,
                                        C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                        C.c_int, C.c_void_p, C.c_int]
        _ref = L
    return _ref


def _p(a):
    return a.ctypes.data if a is not None else None


def mm_f8(lib, x, w, s, rows, cols, br, bc):
    """y[T][rows] by the oracle (lib=oracle()) or the reference (lib=ref())."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
    T = x.shape[0]
    y = np.empty((T, rows), np.float32)
    f = lib.or_mm_f8 if hasattr(lib, "or_mm_f8") else lib.ref_mm
    f(y.ctypes.data, x.ctypes.data, T, w.ctypes.data, s.ctypes.data, rows, cols, br, bc)
    return y


def expert_table(mats_by_e, NE):
    """OrExpert[NE] from {e: [(w, s)] x 3} (missing e: a failed load)."""
    tab = (OrExpert * NE)()
    keep = []
    for e, mats in mats_by_e.items():
        (gw, gs), (uw, us), (dw, ds) = mats
        keep += [gw, gs, uw, us, dw, ds]
        tab[e] = OrExpert(gw.ctypes.data, uw.ctypes.data, dw.ctypes.data, gs.ctypes.data, us.ctypes.data,
                          ds.ctypes.data)
    return tab, keep


def moe(lib, x, sp, router, bias, mats_by_e, shared_mats):
    """Layer output [T][E], idx [T][K], w [T][K] by the oracle or the reference."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, sp.E)
    T = x.shape[0]
    out = np.zeros((T, sp.E), np.float32)
    tab, keep = expert_table(mats_by_e, sp.NE)
    sh = None
    if shared_mats is not None:
        sht, keep2 = expert_table({0: shared_mats}, 1)
        keep += keep2
        sh = C.byref(sht[0])
    router = np.ascontiguousarray(router, np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    if hasattr(lib, "or_moe"):
        idx = np.zeros((T, sp.K), np.int32)
        w = np.zeros((T, sp.K), np.float32)
        rc = lib.or_moe(out.ctypes.data, x.ctypes.data, T, sp.E, sp.I, sp.NE, sp.K, sp.br, sp.bc, sp.norm_topk,
                        sp.routed_scale, sp.limit, router.ctypes.data, bias.ctypes.data, C.addressof(tab),
                        sh, idx.ctypes.data, w.ctypes.data)
        assert rc == 0
        return out, idx, w
    lib.ref_moe(out.ctypes.data, x.ctypes.data, T, sp.E, sp.I, sp.NE, sp.K, sp.br, sp.bc, sp.norm_topk,
                sp.routed_scale, sp.limit, router.ctypes.data, bias.ctypes.data, C.addressof(tab), sh)
    return out, None, None


def router(lib, x, sp, router_w, bias):
    x = np.ascontiguousarray(x, np.float32).reshape(-1, sp.E)
    T = x.shape[0]
    idx = np.zeros((T, sp.K), np.int32)
    w = np.zeros((T, sp.K), np.float32)
    rw = np.ascontiguousarray(router_w, np.float32)
    b = np.ascontiguousarray(bias, np.float32)
    for t in range(T):
        xt = np.ascontiguousarray(x[t])
        if hasattr(lib, "or_router"):
            rc = lib.or_router(idx[t].ctypes.data, w[t].ctypes.data, xt.ctypes.data, rw.ctypes.data, b.ctypes.data,
                               sp.NE, sp.E, sp.K, sp.norm_topk, sp.routed_scale)
            assert rc == 0
        else:
            lib.ref_router(idx[t].ctypes.data, w[t].ctypes.data, xt.ctypes.data, sp.E, sp.NE, sp.K, sp.norm_topk,
                           sp.routed_scale, rw.ctypes.data, b.ctypes.data)
    return idx, w


def _lcg():
    L = oracle()
    L.or_lcg.argtypes = [C.POINTER(C.c_uint32), C.c_void_p, C.c_long]
    state = C.c_uint32(12345)

    def draw(n):
        out = np.empty(max(n, 0), np.uint32)
        if n > 0:
            L.or_lcg(C.byref(state), out.ctypes.data, n)
        return out
    return draw


def _kat_all():
    """Every known-answer case of the reference's test_fp8 main() (tests/unit/test_fp8.c:150-161),
    drawn from its one LCG stream in the reference's order (tests/unit/test_fp8.c:41-54, 74-79,
    113-117): five FP8 matvecs, three int4 matvecs, one int4 quantisation."""
    draw = _lcg()
    fp8 = []
    for rows, cols, br, bc, with_nan in [(2048, 4096, 128, 128, 0), (4096, 2048, 128, 128, 0),
                                         (37, 1021, 16, 128, 0), (9, 13, 4, 4, 0), (64, 256, 128, 64, 1)]:
        srows, scols = (rows + br - 1) // br, (cols + bc - 1) // bc
        n = rows * cols
        w = np.arange(n, dtype=np.uint64)
        w[256:] = draw(n - 256)
        w = (w & 0xff).astype(np.uint8)
        if not with_nan:
            nan = (w & 0x7f) == 0x7f
            w[nan] ^= 1
        s = (draw(srows * scols) % 1000 + 1).astype(np.float32) * np.float32(1e-6)
        x = ((draw(cols) % 20001).astype(np.int64) - 10000).astype(np.float32) * np.float32(1e-4)
        fp8.append(dict(rows=rows, cols=cols, br=br, bc=bc, with_nan=with_nan, w=w, s=s.astype(np.float32),
                        x=x.astype(np.float32)))
    i4 = []
    for rows, cols in [(2048, 4096), (4096, 2048), (9, 128)]:
        groups = cols // 64
        q = (draw(rows * (cols // 2)) & 0xff).astype(np.uint8)
        st = (draw(rows * groups) % 1000 + 1).astype(np.float32) * np.float32(1e-6)
        x = ((draw(cols) % 20001).astype(np.int64) - 10000).astype(np.float32) * np.float32(1e-4)
        i4.append(dict(rows=rows, cols=cols, q=q, steps=st.astype(np.float32), x=x.astype(np.float32)))
    rows, cols, br, bc = 512, 4096, 128, 128
    w = (draw(rows * cols) & 0xff).astype(np.uint8)
    nan = (w & 0x7f) == 0x7f
    w[nan] ^= 1
    srows, scols = (rows + br - 1) // br, (cols + bc - 1) // bc
    s = (draw(srows * scols) % 500 + 1).astype(np.float32) * np.float32(1e-5)
    quant = dict(rows=rows, cols=cols, br=br, bc=bc, w=w, s=s.astype(np.float32))
    return fp8, i4, quant


def fp8_kat_cases():
    """The five FP8 matvec cases of the reference's test_fp8 main() (tests/unit/test_fp8.c:150-157),
    with the reference's own inputs (tests/unit/test_fp8.c:41-54): one LCG stream
    (rng = rng*1664525 + 1013904223 from 12345, next() = rng >> 8) consumed in the reference's
    order; codes are the element index for the first 256 and next() after, NaN codes (low seven
    bits all ones) flipped unless the case keeps them; scales (next()%1000+1)*1e-6f; x
    ((next()%20001) - 10000)*1e-4f."""
    return _kat_all()[0]


def i4_kat_cases():
    """(int4 matvec cases, int4 quantiser case) of the same stream (tests/unit/test_fp8.c:158-161):
    levels are random bytes, steps (next()%1000+1)*1e-6f, x as above; the quantiser's FP8 codes are
    next() with NaN codes flipped and its 128x128 scales (next()%500+1)*1e-5f."""
    _, i4, quant = _kat_all()
    return i4, quant


def mm_i4(lib, x, q, steps, rows, cols):
    """y[T][rows] of an int4 matrix (groups of 64) by the oracle or the reference."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
    T = x.shape[0]
    y = np.empty((T, rows), np.float32)
    q = np.ascontiguousarray(q, np.uint8)
    steps = np.ascontiguousarray(steps, np.float32)
    if hasattr(lib, "or_mm_i4"):
        lib.or_mm_i4(y.ctypes.data, x.ctypes.data, T, q.ctypes.data, steps.ctypes.data, rows, cols, 64)
    else:
        lib.ref_mm_i4(y.ctypes.data, x.ctypes.data, T, q.ctypes.data, steps.ctypes.data, rows, cols)
    return y


def i4_from_f8(lib, w, s, rows, cols, br, bc):
    """(q [rows][cols/2] uint8, steps [rows][cols/64] float32) by the oracle or the reference."""
    q = np.empty((rows, cols // 2), np.uint8)
    st = np.empty((rows, cols // 64), np.float32)
    w = np.ascontiguousarray(w, np.uint8)
    s = np.ascontiguousarray(s, np.float32)
    f = lib.or_i4_from_f8 if hasattr(lib, "or_i4_from_f8") else lib.ref_i4_from_f8
    f(q.ctypes.data, st.ctypes.data, w.ctypes.data, s.ctypes.data, rows, cols, br, bc)
    return q, st


def quantise_expert(lib, mats, sp):
    """[(q, steps)] x 3 of an FP8 expert [(w, s)] x 3 (gate [I][E], up [I][E], down [E][I])."""
    shapes = [(sp.I, sp.E), (sp.I, sp.E), (sp.E, sp.I)]
    return [i4_from_f8(lib, w, s, r, c, sp.br, sp.bc) for (w, s), (r, c) in zip(mats, shapes)]


def moe_i4(lib, x, sp, router, bias, qmats_by_e, shared_mats):
    """Layer output [T][E] with int4 routed experts {e: [(q, steps)] x 3} and the FP8 shared
    expert, by the oracle (with idx, w) or the reference (idx, w None)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, sp.E)
    T = x.shape[0]
    out = np.zeros((T, sp.E), np.float32)
    tab, keep = expert_table(qmats_by_e, sp.NE)
    sh = None
    if shared_mats is not None:
        sht, keep2 = expert_table({0: shared_mats}, 1)
        keep += keep2
        sh = C.byref(sht[0])
    router = np.ascontiguousarray(router, np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    if hasattr(lib, "or_moe_i4"):
        idx = np.zeros((T, sp.K), np.int32)
        w = np.zeros((T, sp.K), np.float32)
        rc = lib.or_moe_i4(out.ctypes.data, x.ctypes.data, T, sp.E, sp.I, sp.NE, sp.K, sp.br, sp.bc, sp.norm_topk,
                           sp.routed_scale, sp.limit, router.ctypes.data, bias.ctypes.data, C.addressof(tab),
                           sh, idx.ctypes.data, w.ctypes.data)
        assert rc == 0
        return out, idx, w
    lib.ref_moe_i4(out.ctypes.data, x.ctypes.data, T, sp.E, sp.I, sp.NE, sp.K, sp.br, sp.bc, sp.norm_topk,
                   sp.routed_scale, sp.limit, router.ctypes.data, bias.ctypes.data, C.addressof(tab), sh)
    return out, None, None


def ref_proto(sp, x, router, bias, mats_by_e, shared_mats, layer, next_router, next_bias, prefetch_n, prefill_next,
              with_hint=True, with_getmany=True):
    """The reference glm53f_moe's output and its recorded expert-source calls (ref_shim.c
    ref_moe_proto): [1, L, e] get, [2, L, e] release, [3, L, n, ids] getmany, [4, L, n, ids] hint."""
    R = ref()
    x = np.ascontiguousarray(x, np.float32).reshape(-1, sp.E)
    T = x.shape[0]
    out = np.zeros((T, sp.E), np.float32)
    tab, keep = expert_table(mats_by_e, sp.NE)
    sht, keep2 = expert_table({0: shared_mats}, 1)
    router = np.ascontiguousarray(router, np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    nr = np.ascontiguousarray(next_router, np.float32)
    nb = np.ascontiguousarray(next_bias, np.float32)
    log = np.zeros(1 << 20, np.int32)
    n = R.ref_moe_proto(out.ctypes.data, x.ctypes.data, T, sp.E, sp.I, sp.NE, sp.K, sp.br, sp.bc, sp.norm_topk,
                        sp.routed_scale, sp.limit, router.ctypes.data, bias.ctypes.data, C.addressof(tab),
                        C.byref(sht[0]), layer, nr.ctypes.data, nb.ctypes.data, prefetch_n, prefill_next,
                        int(with_hint), int(with_getmany), log.ctypes.data, len(log))
    assert n >= 0
    return out, log[:n].copy()
