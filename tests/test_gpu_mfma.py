"""GPU parity of the MFMA-tiled decode kernel (k_dec_mfma, T = 1) and its layout conversion.

Bar (the path's stated tolerance): routing indices and weights bit-exact against the C oracle
(src/core/glm53f_ops.c:945-976); every output element within 1e-2 absolute + 2e-3 relative of
the oracle's output for the same inputs (src/core/glm53f_ops.c:185-228, 486-494, 1329-1340).
The kernel multiplies on the FP8 matrix cores with fp32 accumulation; its inputs are split into
E4M3 planes (exact for bf16-valued x, about 12 bits for the SwiGLU activations)."""
import ctypes as C

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
import oracle_lib as O
from glm53h import DevBuf, check
from test_gpu_grouped import within
from test_gpu_parity import run_layer, same, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


def oracle_check(layer, x, out, idx, w, what, drop=()):
    sp = layer.sp
    mats = {int(e): layer.fetch_expert(int(e)) for e in idx[0] if int(e) not in drop}
    sh = layer.fetch_expert("shared") if sp.shared else None
    want, wi, ww = O.moe(O.oracle(), x, sp, layer.router_f32, layer.bias_f32, mats, sh)
    assert np.array_equal(idx, wi) and same(w, ww), what
    within(out, want, what)
    return want


@pytest.mark.parametrize("rows,cols", [(2048, 4096), (4096, 2048), (8, 128), (24, 384)])
def test_mtile_device_equals_host(L, rows, cols):
    say("mtile", rows, cols)
    rng = np.random.default_rng(rows + 3 * cols)
    a = rng.integers(0, 256, rows * cols, dtype=np.uint8)
    src, dst, back = DevBuf.from_array(a), DevBuf(a.nbytes), DevBuf(a.nbytes)
    check(L.g53h_mtile_f8(dst.ptr, src.ptr, rows, cols, 0), "mtile")
    check(L.g53h_mtile_f8(back.ptr, dst.ptr, rows, cols, 1), "unmtile")
    want = np.empty_like(a)
    assert L.g53h_mtile_f8_host(want.ctypes.data, a.ctypes.data, rows, cols, 0) == 0
    assert np.array_equal(dst.download(np.uint8), want)
    assert np.array_equal(back.download(np.uint8), a)


@pytest.fixture(scope="module")
def mlayer(L):
    say("building the config-2 layer, MFMA-tiled")
    return S.DeviceLayer.build(S.spec(2), mfma=True)


def test_mfma_decode_config2(L, mlayer):
    sp = mlayer.sp
    for t in range(4):
        x = S.x_host(sp, 1, batch=40 + t)
        say("mfma decode config 2, token", t)
        out, idx, w = run_layer(mlayer, x, 1)
        assert L.g53h_decode_errors() == 0
        oracle_check(mlayer, x, out, idx, w, f"config 2 token {t}")


def test_mfma_decode_golden_router(L, mlayer):
    """The committed config-2 golden routing (compiled reference) through the MFMA kernel."""
    import os
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))
    sp = mlayer.sp
    x = S.x_host(sp, 64, batch=0)
    for t in (0, 17, 63):
        _, idx, w = run_layer(mlayer, x[t:t + 1], 1)
        assert np.array_equal(idx[0], gold["c2r_idx"][t])
        assert same(w[0], gold["c2r_w"][t])


def test_mfma_decode_is_deterministic(L, mlayer):
    sp = mlayer.sp
    x = S.x_host(sp, 1, batch=90)
    o1, i1, _ = run_layer(mlayer, x, 1)
    for _ in range(3):
        o2, i2, _ = run_layer(mlayer, x, 1)
        assert np.array_equal(i1, i2) and np.array_equal(o1.view(np.uint32), o2.view(np.uint32))


def test_mfma_decode_routed_given(L, mlayer):
    """g53h_moe_routed_given skips the routing: the same output as the routed call."""
    sp = mlayer.sp
    x = S.x_host(sp, 1, batch=91)
    out, idx, w = run_layer(mlayer, x, 1)
    xd, o2 = DevBuf.from_array(x), DevBuf(sp.E * 4)
    idd, wd = DevBuf.from_array(idx), DevBuf.from_array(w)
    check(L.g53h_moe_routed_given(o2.ptr, xd.ptr, 1, C.byref(mlayer.layer), idd.ptr, wd.ptr), "given")
    glm53h.sync()
    assert np.array_equal(o2.download(np.float32).reshape(1, sp.E).view(np.uint32), out.view(np.uint32))


@pytest.mark.parametrize("NE,K,shared,norm", [(512, 4, False, 1), (288, 15, True, 1), (640, 8, True, 0)])
def test_mfma_decode_other_layouts(L, NE, K, shared, norm):
    sp = S.spec(2, NE=NE, K=K, shared=shared, norm_topk=norm, seed=11)
    say("mfma decode layout NE", NE, "K", K, "shared", shared, "norm_topk", norm)
    layer = S.DeviceLayer.build(sp, mfma=True)
    for t in range(2):
        x = S.x_host(sp, 1, batch=20 + t)
        out, idx, w = run_layer(layer, x, 1)
        assert L.g53h_decode_errors() == 0
        oracle_check(layer, x, out, idx, w, f"NE {NE} K {K} token {t}")
    del layer


def test_mfma_decode_clamp_half_and_large_inputs(L):
    """SwiGLU limit 0.5 (the reference's glm_tiny fixture value) and inputs scaled by 1000 (the
    per-32-value plane scales follow the data)."""
    sp = S.spec(2, NE=64, limit=0.5, seed=13)
    layer = S.DeviceLayer.build(sp, mfma=True)
    x = S.x_host(sp, 1, batch=5)
    out, idx, w = run_layer(layer, x, 1)
    oracle_check(layer, x, out, idx, w, "limit 0.5")
    xb = (x * 1024.0).astype(np.float32)
    out, idx, w = run_layer(layer, xb, 1)
    oracle_check(layer, xb, out, idx, w, "x * 1024")
    assert L.g53h_decode_errors() == 0


def test_mfma_decode_absent_and_unusable_experts(L):
    """A routed expert without codes contributes zero (the reference's drop path); one that is
    not MFMA-tiled, or has other blocks, is flagged (bit 8) and contributes zero too."""
    sp = S.spec(2, seed=12)
    layer = S.DeviceLayer.build(sp, mfma=True)
    x = S.x_host(sp, 1, batch=30)
    _, idx, _ = run_layer(layer, x, 1)
    gone, bad, other = int(idx[0][2]), int(idx[0][5]), int(idx[0][7])
    say("mfma decode with expert", gone, "absent,", bad, "unusable and", other, "octet-tiled")
    descs = (glm53h.G53hExpert * (sp.NE + 1)).from_buffer_copy(bytes(layer.experts))
    descs[gone].gate.w = None
    descs[bad].up.bc = 64
    descs[other].down.flags = 2
    table = DevBuf.from_array(np.frombuffer(bytes(descs), np.uint8))
    lay = glm53h.G53hMoeLayer.from_buffer_copy(bytes(layer.layer))
    lay.experts = table.ptr
    lay.shared = table.ptr + sp.NE * C.sizeof(glm53h.G53hExpert)
    xd = DevBuf.from_array(x)
    out, idd, wd = DevBuf(sp.E * 4), DevBuf(sp.K * 4), DevBuf(sp.K * 4)
    check(L.g53h_moe(out.ptr, xd.ptr, 1, C.byref(lay), idd.ptr, wd.ptr), "g53h_moe")
    glm53h.sync()
    assert L.g53h_decode_errors() == 8
    oracle_check(layer, x, out.download(np.float32).reshape(1, sp.E), idd.download(np.int32).reshape(1, sp.K),
                 wd.download(np.float32).reshape(1, sp.K), "drops", drop=(gone, bad, other))


def test_mfma_layer_refuses_batches(L, mlayer):
    """MFMA-tiled experts are read by the single-token kernel only: a batch is refused with an
    error, not computed from the wrong byte order."""
    sp = mlayer.sp
    x = S.x_host(sp, 2, batch=3)
    xd, out = DevBuf.from_array(x), DevBuf(2 * sp.E * 4)
    rc = L.g53h_moe(out.ptr, xd.ptr, 2, C.byref(mlayer.layer), None, None)
    assert rc != 0
    assert b"tiled" in glm53h.lib().g53h_error()
