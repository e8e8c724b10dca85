"""GPU parity of the int4 decode on the FP4 matrix cores (k_dec_mfma over int4 MFMA-tiled routed
experts, G53H_MAT_I4 | G53H_MAT_MTILED; the reference's --experts int4 mode at T = 1) and of its
layout conversion.

Bar (the path's stated tolerance, as for the FP8 matrix-core decode): routing indices and weights
bit-exact against the C oracle (src/core/glm53f_ops.c:945-976); every output element within
1e-2 absolute + 2e-3 relative of the oracle's output for the same int4 experts
(src/core/glm53f_ops.c:236-296 matmul_i4, the shared expert FP8 :185-228, the combine
:1329-1340), and of the compiled reference's golden config-2 output (tests/golden/i4.npz). The
kernel takes the levels as two FP4 planes and a constant one, exactly; the inputs as E4M3 planes
(exact for bf16-valued x, about 12 bits for the SwiGLU activations); fp32 accumulation."""
import ctypes as C
import os

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
import oracle_lib as O
from glm53h import DevBuf, check
from test_gpu_grouped import within
from test_gpu_parity import run_layer, same, say

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
G4 = np.load(os.path.join(HERE, "golden", "i4.npz"))


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


@pytest.fixture(scope="module")
def layer(L):
    say("building the config-2 layer: int4 routed experts MFMA-tiled, FP8 shared expert MFMA-tiled")
    return S.DeviceLayer.build(S.spec(2), i4=True, mfma=True)


@pytest.mark.parametrize("rows,cols", [(2048, 4096), (4096, 2048), (8, 128), (24, 384)])
def test_mtile_i4_device_equals_host(L, rows, cols):
    say("int4 mtile", rows, cols)
    rng = np.random.default_rng(rows + 5 * cols)
    a = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    st = rng.standard_normal(rows * (cols // 64)).astype(np.float32)
    src, ss = DevBuf.from_array(a), DevBuf.from_array(st)
    dst, ds, back, bs = DevBuf(a.nbytes), DevBuf(st.nbytes), DevBuf(a.nbytes), DevBuf(st.nbytes)
    check(L.g53h_mtile_i4(dst.ptr, ds.ptr, src.ptr, ss.ptr, rows, cols, 0), "mtile_i4")
    check(L.g53h_mtile_i4(back.ptr, bs.ptr, dst.ptr, ds.ptr, rows, cols, 1), "unmtile_i4")
    want, wants = np.zeros_like(a), np.zeros_like(st)
    assert L.g53h_mtile_i4_host(want.ctypes.data, wants.ctypes.data, a.ctypes.data, st.ctypes.data, rows, cols, 0) == 0
    assert np.array_equal(dst.download(np.uint8), want)
    assert np.array_equal(ds.download(np.float32).view(np.uint32), wants.view(np.uint32))
    assert np.array_equal(back.download(np.uint8), a)
    assert np.array_equal(bs.download(np.float32).view(np.uint32), st.view(np.uint32))


def oracle_check(layer, x, out, idx, w, what):
    sp = layer.sp
    qm = {int(e): layer.fetch_expert(int(e)) for e in idx[0]}
    want, wi, ww = O.moe_i4(O.oracle(), x, sp, layer.router_f32, layer.bias_f32, qm, layer.fetch_expert("shared"))
    assert np.array_equal(idx, wi) and same(w, ww), what
    within(out, want, what)


def test_i4mfma_decode_golden(L, layer):
    """The compiled reference's config-2 int4 output (its own quantisation of the same experts)."""
    sp = layer.sp
    assert L.g53h_decode_errors() == 0
    say("int4 matrix-core decode, config 2, against the compiled reference's output")
    out, _, _ = run_layer(layer, S.x_host(sp, 1, batch=0), 1)
    assert L.g53h_decode_errors() == 0
    within(out[0], G4["c2_out"], "config 2 against the reference")


def test_i4mfma_decode_tokens(L, layer):
    sp = layer.sp
    x = S.x_host(sp, 4, batch=11)
    for t in range(4):
        say("int4 matrix-core decode, config 2, token", t)
        out, idx, w = run_layer(layer, x[t:t + 1], 1)
        assert L.g53h_decode_errors() == 0
        oracle_check(layer, x[t:t + 1], out, idx, w, f"config 2 int4 token {t}")


def test_i4mfma_levels_roundtrip(L, layer):
    """The tiled levels and steps in HBM are the quantiser's, element for element."""
    sp = layer.sp
    e = 17
    d = layer.experts[e]
    for m in (d.gate, d.up, d.down):
        assert m.flags == 4 | 8 and m.bc == 64
    got = layer.fetch_expert(e)
    # the same expert quantised again into a row-major int4 layer
    say("building the config-2 layer, int4 row-major, to compare one expert")
    rm = S.DeviceLayer.build(S.spec(2), i4=True)
    for (wt, stt), (wr, sr) in zip(got, rm.fetch_expert(e)):
        assert np.array_equal(wt, wr) and np.array_equal(stt.view(np.uint32), sr.view(np.uint32))


def test_i4mfma_routing_given_and_batches_refused(L, layer):
    sp = layer.sp
    x = S.x_host(sp, 1, batch=12)
    out, idx, w = run_layer(layer, x, 1)
    say("int4 matrix-core decode with the routing given")
    xd, o2 = DevBuf.from_array(x), DevBuf(sp.E * 4)
    gi, gw = DevBuf.from_array(idx[0].copy()), DevBuf.from_array(w[0].copy())
    check(glm53h.lib().g53h_moe_routed_given(o2.ptr, xd.ptr, 1, C.byref(layer.layer), gi.ptr, gw.ptr), "given")
    glm53h.sync()
    assert same(o2.download(np.float32), out[0])
    x2 = DevBuf.from_array(S.x_host(sp, 2, batch=12))
    out2 = DevBuf(2 * sp.E * 4)
    assert glm53h.lib().g53h_moe(out2.ptr, x2.ptr, 2, C.byref(layer.layer), None, None) != 0
    glm53h.sync()
    assert L.g53h_decode_errors() == 0
