"""The CPU oracle (oracle/g53_oracle.c) pinned before it is trusted: against the compiled
reference's golden outputs, the reference's own known-answer inputs, closed forms, brute force
on small inputs and library routines. No GPU needed."""
import ctypes as C
import math
import os

import numpy as np
import pytest

import oracle_lib as O
import glm53h
import glm53h.synth as S

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return np.all((bits(a) == bits(b)) | (np.isnan(a) & np.isnan(b)))


# ------------------------------------------------------------------------- E4M3 ----
def e4m3_closed_form(b):
    s, e, m = b >> 7, (b >> 3) & 15, b & 7
    if e == 15 and m == 7:
        return float("nan")
    v = (m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
    return -v if s else v


def test_e4m3_all_codes_closed_form():
    L = O.oracle()
    for b in range(256):
        want = np.float32(e4m3_closed_form(b))
        assert same([L.or_e4m3f(b)], [want]), b
        assert same([glm53h.lib().glm53f_e4m3f(b)], [want]), b   # the product's host twin


@pytest.mark.skipif(not O.have_ref(), reason="reference not built")
def test_e4m3_matches_reference_table():
    for b in range(256):
        assert same([O.oracle().or_e4m3f(b)], [O.ref().ref_e4m3f(b)])


# ----------------------------------------------------------------- FP8 matvec ----
def test_matvec_known_answer_cases_bit_exact():
    """The reference's test_fp8 inputs; expected outputs are the compiled reference's."""
    for i, c in enumerate(O.fp8_kat_cases()):
        y = O.mm_f8(O.oracle(), c["x"], c["w"], c["s"], c["rows"], c["cols"], c["br"], c["bc"])[0]
        assert same(y, GOLD[f"kat_y{i}"]), (c["rows"], c["cols"])
        if c["with_nan"]:
            assert np.isnan(y).any()


def test_matvec_against_fp64_dequantised_product():
    """|y - W_deq x| within the accumulated float rounding: a transposed scale index, a
    dropped block or a wrong sign fails by orders of magnitude."""
    rng = np.random.default_rng(5)
    for rows, cols, br, bc in [(64, 384, 128, 128), (37, 1021, 16, 128), (9, 13, 4, 4)]:
        w = rng.integers(0, 256, rows * cols).astype(np.uint8)
        w[(w & 0x7f) == 0x7f] ^= 1
        srows, scols = (rows + br - 1) // br, (cols + bc - 1) // bc
        s = rng.uniform(1e-4, 1e-2, srows * scols).astype(np.float32)
        x = rng.standard_normal(cols).astype(np.float32)
        y = O.mm_f8(O.oracle(), x, w, s, rows, cols, br, bc)[0].astype(np.float64)
        dec = np.array([e4m3_closed_form(b) for b in range(256)])[w].reshape(rows, cols)
        S_full = np.repeat(np.repeat(s.reshape(srows, scols), br, 0), bc, 1)[:rows, :cols]
        ref = (dec * S_full) @ x.astype(np.float64)
        mag = np.abs(dec * S_full) @ np.abs(x.astype(np.float64))
        assert np.all(np.abs(y - ref) <= 1e-6 * mag + 1e-30)


def test_matvec_batch_is_per_token():
    rng = np.random.default_rng(6)
    rows, cols = 16, 256
    w = rng.integers(0, 126, rows * cols).astype(np.uint8)
    s = rng.uniform(1e-3, 1e-2, 2).astype(np.float32)
    x = rng.standard_normal((5, cols)).astype(np.float32)
    yb = O.mm_f8(O.oracle(), x, w, s, rows, cols, 128, 128)
    for t in range(5):
        assert same(yb[t], O.mm_f8(O.oracle(), x[t], w, s, rows, cols, 128, 128)[0])


# ---------------------------------------------------------------------- SwiGLU ----
def test_swiglu_closed_form():
    g = np.array([-50, -3, -0.5, 0, 0.5, 3, 9.99, 10, 12, 1e4], np.float32)
    u = np.array([3, -20, 0.25, 5, -0.5, 11, -11, 2, 2, -3], np.float32)
    y = np.empty(len(g), np.float32)
    gu = np.concatenate([g, u])
    O.oracle().or_swiglu(y.ctypes.data, gu.ctypes.data, len(g), C.c_float(10.0))
    gi = np.minimum(g.astype(np.float64), 10)
    ui = np.clip(u.astype(np.float64), -10, 10)
    want = gi / (1 + np.exp(-gi)) * ui
    assert np.allclose(y, want, rtol=1e-6, atol=1e-30)
    assert abs(y[-1] - 10 / (1 + math.exp(-10)) * -3) < 1e-4     # both clamps bind


# ---------------------------------------------------------------------- router ----
def brute_router(x, W, b, K, norm, scale):
    score = 1 / (1 + np.exp(-(W.astype(np.float64) @ x.astype(np.float64))))
    choice = score + b
    order = sorted(range(len(b)), key=lambda e: (-choice[e], e))[:K]
    w = score[order]
    if norm:
        w = w / (w.sum() + 1e-20)
    return np.array(order), w * scale


def test_router_brute_force_small():
    sp = S.spec(1)
    W, b = S.router_host(sp), S.bias_host(sp)
    x = S.x_host(sp, 16, batch=7)
    idx, w = O.router(O.oracle(), x, sp, W, b)
    for t in range(16):
        bi, bw = brute_router(x[t], W, b, sp.K, sp.norm_topk, sp.routed_scale)
        assert list(idx[t]) == list(bi)
        assert np.allclose(w[t], bw, rtol=1e-5)


def test_router_ties_pick_lowest_index():
    sp = S.LayerSpec(E=8, I=8, NE=6, K=3)
    W = np.zeros((6, 8), np.float32)                  # every score sigmoid(0) = 0.5
    b = np.array([0.1, 0.3, 0.3, 0.0, 0.3, 0.1], np.float32)
    idx, w = O.router(O.oracle(), np.ones(8, np.float32), sp, W, b)
    assert list(idx[0]) == [1, 2, 4]
    assert np.allclose(w[0], [2.5 / 3] * 3)


def test_router_golden():
    sp1, sp2 = S.spec(1), S.spec(2)
    idx, w = O.router(O.oracle(), S.x_host(sp1, 8), sp1, S.router_host(sp1), S.bias_host(sp1))
    assert np.array_equal(idx, GOLD["c1_idx"]) and same(w, GOLD["c1_w"])
    idx, w = O.router(O.oracle(), S.x_host(sp2, 64), sp2, S.router_host(sp2), S.bias_host(sp2))
    assert np.array_equal(idx, GOLD["c2r_idx"]) and same(w, GOLD["c2r_w"])


def test_route_topn_nan_rules():
    L = O.oracle()
    L.or_route_topn.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int]
    E = 4
    x = np.ones(E, np.float32)
    W = np.zeros((5, E), np.float32)
    for b, want in [([0.1, 0.5, 0.2, 0.5, 0.0], [1, 3, 2]),
                    ([np.nan, 0.5, 0.2, 0.3, 0.0], [0, 1, 3]),        # NaN at 0 wins first
                    ([0.1, np.nan, 0.2, 0.3, 0.0], [3, 2, 0])]:       # NaN elsewhere skipped
        b = np.array(b, np.float32)
        idx = np.zeros(3, np.int32)
        L.or_route_topn(idx.ctypes.data, 3, x.ctypes.data, W.ctypes.data, b.ctypes.data, 5, E)
        assert list(idx) == want, b


# ------------------------------------------------------------------------- MoE ----
def c1_inputs():
    sp = S.spec(1)
    return sp, S.router_host(sp), S.bias_host(sp), {e: S.expert_host(sp, e) for e in range(sp.NE)}, \
        S.expert_host(sp, "shared")


def test_moe_config1_golden():
    sp, W, b, mats, sh = c1_inputs()
    x = S.x_host(sp, 8, batch=0)
    out, idx, w = O.moe(O.oracle(), x, sp, W, b, mats, sh)
    assert same(out, GOLD["c1_out"]) and np.array_equal(idx, GOLD["c1_idx"])
    xb = S.x_host(sp, 5, batch=1)
    assert same(O.moe(O.oracle(), xb, sp, W, b, mats, sh)[0], GOLD["c1b_out"])
    assert same(O.moe(O.oracle(), xb, sp, W, b, mats, None)[0], GOLD["c1b_routed_out"])
    drop = {e: m for e, m in mats.items() if e not in (3, 7)}
    assert same(O.moe(O.oracle(), xb, sp, W, b, drop, sh)[0], GOLD["c1d_out"])


def run_expert(sp, x, mats):
    """gate, up, SwiGLU, down of one expert through the oracle's unit functions."""
    (gw, gs), (uw, us), (dw, ds) = mats
    g = O.mm_f8(O.oracle(), x, gw, gs, sp.I, sp.E, sp.br, sp.bc)[0]
    u = O.mm_f8(O.oracle(), x, uw, us, sp.I, sp.E, sp.br, sp.bc)[0]
    a = np.empty(sp.I, np.float32)
    gu = np.concatenate([g, u])
    O.oracle().or_swiglu(a.ctypes.data, gu.ctypes.data, sp.I, C.c_float(sp.limit))
    return O.mm_f8(O.oracle(), a, dw, ds, sp.E, sp.I, sp.br, sp.bc)[0]


def test_moe_combine_is_weighted_sum_of_experts():
    """The layer equals sum_j w_j expert_j(x) + shared(x), each expert run on its own
    (a dropped term, a wrong weight index or a missing shared expert fails)."""
    sp, W, b, mats, sh = c1_inputs()
    x = S.x_host(sp, 1, batch=3)
    out, idx, w = O.moe(O.oracle(), x, sp, W, b, mats, sh)
    acc = np.zeros(sp.E)
    for j, e in enumerate(idx[0]):
        acc += np.float64(w[0][j]) * run_expert(sp, x, mats[int(e)])
    acc += run_expert(sp, x, sh)
    assert np.allclose(out[0], acc, rtol=1e-5, atol=1e-7)


def test_moe_config2_one_token_golden():
    sp = S.spec(2)
    W, b = S.router_host(sp), S.bias_host(sp)
    x = S.x_host(sp, 64)[:1]
    idx, _ = O.router(O.oracle(), x, sp, W, b)
    mats = {int(e): S.expert_host(sp, int(e)) for e in idx[0]}
    out = O.moe(O.oracle(), x, sp, W, b, mats, S.expert_host(sp, "shared"))[0]
    assert same(out[0], GOLD["c2_out"])


def test_moe_glm_tiny_fixture_golden():
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    import tinyst
    t, cfg = tinyst.load(), tinyst.config()
    for L in cfg["moe_layers"]:
        sp = S.LayerSpec(E=cfg["E"], I=cfg["I"], NE=cfg["NE"], K=cfg["K"], norm_topk=cfg["norm_topk"],
                         routed_scale=cfg["routed_scale"], limit=cfg["limit"], br=cfg["br"], bc=cfg["bc"])
        W, b, ex, sh = tinyst.layer(t, L)
        out, idx, w = O.moe(O.oracle(), GOLD[f"tiny{L}_x"], sp, W, b, ex, sh)
        assert same(out, GOLD[f"tiny{L}_out"]) and np.array_equal(idx, GOLD[f"tiny{L}_idx"])


@pytest.mark.skipif(not O.have_ref(), reason="reference not built")
def test_moe_random_cases_against_reference():
    """Fresh seeds (not in the fixtures) through both the oracle and the compiled reference."""
    for seed in (11, 12):
        sp = S.spec(1, seed=seed, limit=0.05)         # a small clamp so it binds
        W, b = S.router_host(sp), S.bias_host(sp)
        mats = {e: S.expert_host(sp, e) for e in range(sp.NE)}
        sh = S.expert_host(sp, "shared")
        x = S.x_host(sp, 7) * 8
        assert same(O.moe(O.oracle(), x, sp, W, b, mats, sh)[0], O.moe(O.ref(), x, sp, W, b, mats, sh)[0])


# ------------------------------------------------------ shared host arithmetic ----
def test_expf_restatement_matches_glibc_sample():
    """The host build of the device expf restatement against glibc expf on 16M inputs spread
    over the whole float range (the GPU test covers all 2^32)."""
    L = glm53h.lib()
    rng = np.random.default_rng(1)
    x = rng.integers(0, 2 ** 32, 1 << 24, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([x, np.float32([0, -0.0, np.inf, -np.inf, np.nan, 88.72, -103.97, 89, -104])])
    y1, y2 = np.empty_like(x), np.empty_like(x)
    L.g53h_expf_host(y1.ctypes.data, x.ctypes.data, x.size)
    O.oracle().or_expf(y2.ctypes.data, x.ctypes.data, x.size)
    assert same(y1, y2)


def test_e4m3_quantiser_matches_torch():
    import importlib.util
    if importlib.util.find_spec("torch") is None:
        pytest.skip("torch not installed")
    import subprocess
    import sys
    # torch runs in a child process: it carries its own HIP runtime, which must not share a
    # process with the library's.
    code = (
        "import numpy as np, torch\n"
        "rng=np.random.default_rng(3)\n"
        "x=np.concatenate([rng.uniform(-460,460,1<<20), rng.standard_normal(1<<20)*0.01,"
        " rng.standard_normal(1<<18)*1e-3, np.arange(-448,448.5,0.0625)]).astype(np.float32)\n"
        "x=np.clip(x,-448,448)\n"
        "q=torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()\n"
        "np.save('/tmp/_g53_q.npy', np.stack([x.view(np.uint32).astype(np.uint64), q.astype(np.uint64)]))\n")
    subprocess.run([sys.executable, "-c", code], check=True)
    arr = np.load("/tmp/_g53_q.npy")
    x = arr[0].astype(np.uint32).view(np.float32)
    want = arr[1].astype(np.uint8)
    got = quantise_host(x)
    assert np.array_equal(got, want)


def quantise_host(x):
    """E4M3 codes of x via the product's host generator path (scale 1): g53_quant(v, 1.0)."""
    import ctypes
    here = os.path.dirname(os.path.abspath(__file__))
    so = os.path.join(here, "..", "glm-5.3-flash-in-c_amd", "lib", "libglm53h.so")
    L = ctypes.CDLL(so)
    f = L.g53h_quant_host
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float]
    out = np.empty(x.size, np.uint8)
    f(out.ctypes.data, np.ascontiguousarray(x).ctypes.data, x.size, ctypes.c_float(1.0))
    return out


def test_synthetic_generator_statistics_and_determinism():
    a = S.normal_host(1 << 20, 7, 99, 1.0, False)
    b = S.normal_host(1 << 20, 7, 99, 1.0, False)
    c = S.normal_host(1 << 20, 8, 99, 1.0, False)
    assert same(a, b) and not same(a, c)
    assert abs(a.mean()) < 5e-3 and abs(a.std() - 1) < 5e-3
    sp = S.spec(1)
    w1, s1 = S.expert_host(sp, 3)[0]
    w2, s2 = S.expert_host(sp, 3)[0]
    assert np.array_equal(w1, w2) and same(s1, s2)
    # absmax rule: every block holds a code of magnitude 448 (0x7e) and no NaN code
    assert ((w1 & 0x7f) == 0x7e).any() and not ((w1 & 0x7f) == 0x7f).any()
