"""GPU parity: the gfx950 path, called through the C ABI, against the oracle and the golden
outputs of the compiled reference. Bar: bit-exact (the decode path reproduces the reference's
rounding step by step), routing indices exact."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
import oracle_lib as O
from glm53h import DevBuf, G53hMat, check

pytestmark = pytest.mark.gpu
GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))


def say(*a):
    print("[gpu]", *a, flush=True)


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


@pytest.fixture(scope="module")
def c2layer(L):
    say("building config-2 layer (288 experts in HBM)")
    return S.DeviceLayer.build(S.spec(2))


def test_e4m3_decode_all_codes(L):
    say("e4m3 decode, 256 codes")
    codes = DevBuf.from_array(np.arange(256, dtype=np.uint8))
    out = DevBuf(256 * 4)
    check(L.g53h_e4m3_decode(out.ptr, codes.ptr, 256), "decode")
    got = out.download(np.float32)
    want = np.array([O.oracle().or_e4m3f(b) for b in range(256)], np.float32)
    assert same(got, want)


def test_expf_all_float_inputs(L):
    """The device expf restatement equals the host's glibc expf on every float."""
    say("expf over all 2^32 inputs")
    chunk = 1 << 28
    buf = DevBuf(chunk * 4)
    host = np.empty(chunk, np.float32)
    first = C.c_long()
    total = 0
    for base in range(0, 1 << 32, chunk):
        check(L.g53h_expf_range(buf.ptr, base, chunk), "expf_range")
        check(L.g53h_d2h(host.ctypes.data, buf.ptr, host.nbytes), "d2h")
        bad = O.oracle().or_expf_mismatches(host.ctypes.data, base, chunk, C.byref(first))
        assert bad == 0, f"{bad} mismatches from base {base:#x}, first at {base + first.value:#x}"
        total += chunk
    assert total == 1 << 32


@pytest.mark.parametrize("shape", [(256, 128, 128, 128), (37, 1021, 16, 128), (9, 13, 4, 4), (2048, 4096, 128, 128)])
def test_synth_device_equals_host(L, shape):
    rows, cols, br, bc = shape
    say("synth", shape)
    srows, scols = (rows + br - 1) // br, (cols + bc - 1) // bc
    w, s = DevBuf(rows * cols), DevBuf(srows * scols * 4)
    check(L.g53h_synth_f8(w.ptr, s.ptr, rows, cols, br, bc, 42, 77, C.c_float(0.02)), "synth")
    wh = np.empty(rows * cols, np.uint8)
    sh = np.empty(srows * scols, np.float32)
    L.g53h_synth_f8_host(wh.ctypes.data, sh.ctypes.data, rows, cols, br, bc, 42, 77, C.c_float(0.02))
    assert np.array_equal(w.download(np.uint8), wh)
    assert same(s.download(np.float32), sh)


def test_matvec_known_answer_cases(L):
    """The reference test_fp8 cases through g53h_mm_f8: bit-identical to the reference."""
    for i, c in enumerate(O.fp8_kat_cases()):
        say("kat", c["rows"], c["cols"], c["br"], c["bc"])
        w, s, x = DevBuf.from_array(c["w"]), DevBuf.from_array(c["s"]), DevBuf.from_array(c["x"])
        y = DevBuf(c["rows"] * 4)
        m = G53hMat(w.ptr, s.ptr, c["rows"], c["cols"], c["br"], c["bc"], (c["cols"] + c["bc"] - 1) // c["bc"], 0)
        check(L.g53h_mm_f8(y.ptr, x.ptr, 1, C.byref(m)), "mm")
        assert same(y.download(np.float32), GOLD[f"kat_y{i}"])


def test_router_config2(L, c2layer):
    """Batches on both matrix-core forms: 16 x 16 tiles (64, 256 tokens) and 32 x 32 tiles over
    column ranges (600 tokens, a partial last tile; 2048, config 4)."""
    sp = c2layer.sp
    for batch, T in [(0, 64), (5, 256), (7, 600), (6, 2048)]:
        say("router config 2", batch, T)
        x = S.x_host(sp, T, batch=batch)
        xd = DevBuf.from_array(x)
        idx, w, flag = DevBuf(T * sp.K * 4), DevBuf(T * sp.K * 4), DevBuf(4)
        flag.zero()
        check(L.g53h_router(idx.ptr, w.ptr, xd.ptr, T, c2layer.router.ptr, 1, c2layer.bias.ptr, sp.NE, sp.E, sp.K,
                            sp.norm_topk, C.c_float(sp.routed_scale), flag.ptr), "router")
        gi, gw = idx.download(np.int32).reshape(T, sp.K), w.download(np.float32).reshape(T, sp.K)
        if batch == 0:
            wi, ww = GOLD["c2r_idx"], GOLD["c2r_w"]
        else:
            wi, ww = O.router(O.oracle(), x, sp, c2layer.router_f32, c2layer.bias_f32)
        assert np.array_equal(gi, wi)
        assert same(gw, ww)
        assert flag.download(np.int32)[0] == 0


def run_layer(layer, x, T):
    sp = layer.sp
    xd = DevBuf.from_array(x)
    out, idx, w = DevBuf(T * sp.E * 4), DevBuf(T * sp.K * 4), DevBuf(T * sp.K * 4)
    layer.forward(out, xd, T, idx, w)
    glm53h.sync()
    return (out.download(np.float32).reshape(T, sp.E), idx.download(np.int32).reshape(T, sp.K),
            w.download(np.float32).reshape(T, sp.K))


def test_layer_config1(L):
    sp = S.spec(1)
    say("config 1 layer")
    layer = S.DeviceLayer.build(sp)
    x = S.x_host(sp, 8, batch=0)
    for t in range(8):                                  # decode, one token per call
        out, idx, _ = run_layer(layer, x[t:t + 1], 1)
        assert np.array_equal(idx[0], GOLD["c1_idx"][t])
        assert same(out[0], GOLD["c1_out"][t]), t
    xb = S.x_host(sp, 5, batch=1)
    out, _, _ = run_layer(layer, xb, 5)                # five tokens in one call
    assert same(out, GOLD["c1b_out"])
    sp_r = S.spec(1, shared=False)
    lr = S.DeviceLayer.build(sp_r)
    out, _, _ = run_layer(lr, xb, 5)
    assert same(out, GOLD["c1b_routed_out"])


@pytest.mark.parametrize("fused", [1, 0])
def test_layer_config2_decode(L, c2layer, fused):
    """Single-token decode at the released shapes, through the one-launch persistent kernel
    (fused=1) and through the multi-kernel path (fused=0)."""
    prev = L.g53h_set_fused_decode(fused)
    try:
        sp = c2layer.sp
        x = S.x_host(sp, 64, batch=0)
        say("config 2 decode token 0 vs golden, fused", fused)
        out, idx, _ = run_layer(c2layer, x[:1], 1)
        assert L.g53h_decode_errors() == 0
        assert np.array_equal(idx[0], GOLD["c2r_idx"][0])
        assert same(out[0], GOLD["c2_out"])
        for t in (1, 2, 3):
            say("config 2 decode token", t, "vs oracle, fused", fused, "grid", L.g53h_decode_grid())
            out, idx, w = run_layer(c2layer, x[t:t + 1], 1)
            assert L.g53h_decode_errors() == 0
            mats = {int(e): c2layer.fetch_expert(int(e)) for e in idx[0]}
            want, wi, ww = O.moe(O.oracle(), x[t:t + 1], sp, c2layer.router_f32, c2layer.bias_f32, mats,
                                 c2layer.fetch_expert("shared"))
            assert np.array_equal(idx, wi) and same(w, ww)
            assert same(out, want)
        say("config 2: 64 decode tokens back to back, routing vs golden")
        xd = DevBuf.from_array(x)
        outs = DevBuf(64 * sp.E * 4)
        idxs = DevBuf(64 * sp.K * 4)
        for t in range(64):
            check(L.g53h_moe(outs.ptr + t * sp.E * 4, xd.ptr + t * sp.E * 4, 1, C.byref(c2layer.layer),
                             idxs.ptr + t * sp.K * 4, None), "g53h_moe")
        glm53h.sync()
        assert L.g53h_decode_errors() == 0
        assert np.array_equal(idxs.download(np.int32).reshape(64, sp.K), GOLD["c2r_idx"])
    finally:
        L.g53h_set_fused_decode(prev)


def test_layer_config2_small_batch(L, c2layer):
    """Four tokens in one call on the exact per-token kernels (grouped path off): each token's
    output equals its decode output, bit for bit."""
    sp = c2layer.sp
    x = S.x_host(sp, 4, batch=9)
    say("config 2, T=4")
    prev = L.g53h_set_grouped(0)
    try:
        out4, _, _ = run_layer(c2layer, x, 4)
    finally:
        L.g53h_set_grouped(prev)
    for t in range(4):
        out1, _, _ = run_layer(c2layer, x[t:t + 1], 1)
        assert same(out4[t], out1[0])


def test_layer_glm_tiny_fixture(L):
    """The reference's glm_tiny weights (4x4 blocks: the generic kernels)."""
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    import tinyst
    t, cfg = tinyst.load(), tinyst.config()
    for Ly in cfg["moe_layers"]:
        say("glm_tiny layer", Ly)
        W, b, ex, sh = tinyst.layer(t, Ly)
        x = GOLD[f"tiny{Ly}_x"]
        out = dropin_moe(cfg_struct(cfg), W, b, ex, sh, x, drop=())
        assert same(out, GOLD[f"tiny{Ly}_out"])


# --------------------------------------------------------------- the C drop-in ----
def cfg_struct(c):
    cf = glm53h.Glm53fCfg()
    cf.hidden, cf.moe_inter, cf.n_experts, cf.topk, cf.n_shared = c["E"], c["I"], c["NE"], c["K"], 1
    cf.routed_scale, cf.norm_topk, cf.swiglu_limit = c["routed_scale"], c["norm_topk"], c["limit"]
    cf.fp8_block_r, cf.fp8_block_c = c["br"], c["bc"]
    return cf


def fmat(w, s, rows, cols, br, bc):
    return glm53h.Glm53fMat(w.ctypes.data, s.ctypes.data, glm53h.GLM53F_WF8, rows, cols, br, bc,
                            (cols + bc - 1) // bc)


class HostSrc:
    """An Glm53fExpertSrc serving host memory, recording the protocol (get/release/hint)."""

    def __init__(self, cf, experts, drop=()):
        self.cf, self.ex, self.drop = cf, experts, set(drop)
        self.gets, self.releases, self.hints, self.pinned, self.max_pinned = [], [], [], 0, 0
        self.src = glm53h.Glm53fExpertSrc()
        self._get = glm53h.GET_FN(self.get)
        self._rel = glm53h.RELEASE_FN(self.release)
        self.src.get, self.src.release = self._get, self._rel

    def get(self, selfp, layer, e, q):
        self.gets.append(e)
        if e in self.drop:
            return -1
        (gw, gs), (uw, us), (dw, ds) = self.ex[e]
        E, I, br, bc = self.cf.hidden, self.cf.moe_inter, self.cf.fp8_block_r, self.cf.fp8_block_c
        q[0].gate, q[0].up, q[0].down = fmat(gw, gs, I, E, br, bc), fmat(uw, us, I, E, br, bc), fmat(dw, ds, E, I, br, bc)
        self.pinned += 1
        self.max_pinned = max(self.max_pinned, self.pinned)
        return 0

    def release(self, selfp, layer, e):
        self.releases.append(e)
        self.pinned -= 1


def dropin_moe(cf, W, b, ex, sh, x, drop=(), shared=True, src=None, forget=True):
    L = glm53h.lib()
    src = src or HostSrc(cf, ex, drop)
    w = glm53h.Glm53fMoeW()
    Wc, bc_ = np.ascontiguousarray(W, np.float32), np.ascontiguousarray(b, np.float32)
    w.gate, w.bias = Wc.ctypes.data, bc_.ctypes.data
    E, I, br, bcol = cf.hidden, cf.moe_inter, cf.fp8_block_r, cf.fp8_block_c
    (gw, gs), (uw, us), (dw, ds) = sh
    w.sh_gate, w.sh_up, w.sh_down = fmat(gw, gs, I, E, br, bcol), fmat(uw, us, I, E, br, bcol), fmat(dw, ds, E, I, br, bcol)
    w.src = C.pointer(src.src)
    x = np.ascontiguousarray(x, np.float32)
    T = x.shape[0]
    out = np.zeros((T, E), np.float32)
    fn = L.glm53f_moe if shared else L.glm53f_moe_routed
    fn(out.ctypes.data, x.ctypes.data, C.byref(w), C.byref(cf), T, None)
    if forget:
        L.glm53f_forget_host_weights()        # the arrays above are freed after this call
    assert src.pinned == 0
    return out


def test_dropin_moe_config1_host_experts(L):
    sp = S.spec(1)
    cf = cfg_struct(dict(E=sp.E, I=sp.I, NE=sp.NE, K=sp.K, routed_scale=sp.routed_scale, norm_topk=sp.norm_topk,
                         limit=sp.limit, br=sp.br, bc=sp.bc))
    W, b = S.router_host(sp), S.bias_host(sp)
    ex = {e: S.expert_host(sp, e) for e in range(sp.NE)}
    sh = S.expert_host(sp, "shared")
    xb = S.x_host(sp, 5, batch=1)
    say("drop-in glm53f_moe, config 1, T=5")
    src = HostSrc(cf, ex)
    assert same(dropin_moe(cf, W, b, ex, sh, xb, src=src), GOLD["c1b_out"])
    assert src.max_pinned <= sp.K                   # never more pinned than a topk+1 cache allows
    assert sorted(src.gets) == sorted(src.releases)
    say("drop-in glm53f_moe_routed")
    assert same(dropin_moe(cf, W, b, ex, sh, xb, shared=False), GOLD["c1b_routed_out"])
    say("drop-in with experts 3 and 7 failing to load")
    drops0 = C.c_long.in_dll(glm53h.lib(), "glm53f_expert_drops").value
    assert same(dropin_moe(cf, W, b, ex, sh, xb, drop=(3, 7)), GOLD["c1d_out"])
    assert C.c_long.in_dll(glm53h.lib(), "glm53f_expert_drops").value > drops0


def test_dropin_router_and_mm(L):
    sp = S.spec(2)
    W, b = S.router_host(sp), S.bias_host(sp)
    x = S.x_host(sp, 64, batch=0)
    cf = cfg_struct(dict(E=sp.E, I=sp.I, NE=sp.NE, K=sp.K, routed_scale=sp.routed_scale, norm_topk=sp.norm_topk,
                         limit=sp.limit, br=sp.br, bc=sp.bc))
    w = glm53h.Glm53fMoeW()
    w.gate, w.bias = W.ctypes.data, b.ctypes.data
    say("drop-in glm53f_router x 8")
    for t in range(8):
        idx, wt = np.zeros(sp.K, np.int32), np.zeros(sp.K, np.float32)
        xt = np.ascontiguousarray(x[t])
        glm53h.lib().glm53f_router(idx.ctypes.data, wt.ctypes.data, xt.ctypes.data, C.byref(w), C.byref(cf))
        assert np.array_equal(idx, GOLD["c2r_idx"][t]) and same(wt, GOLD["c2r_w"][t])
    glm53h.lib().glm53f_forget_host_weights()
    say("drop-in glm53f_mm on the known-answer cases")
    for i, c in enumerate(O.fp8_kat_cases()):
        m = fmat(c["w"], c["s"], c["rows"], c["cols"], c["br"], c["bc"])
        y = np.zeros(c["rows"], np.float32)
        glm53h.lib().glm53f_mm(y.ctypes.data, c["x"].ctypes.data, C.byref(m))
        assert same(y, GOLD[f"kat_y{i}"])


def test_zero_tokens_is_a_no_op(L, c2layer):
    out = DevBuf(16)
    check(glm53h.lib().g53h_moe(out.ptr, out.ptr, 0, C.byref(c2layer.layer), None, None), "T=0")
