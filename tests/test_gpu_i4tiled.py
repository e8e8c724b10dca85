"""GPU parity of the one-launch int4 decode (k_dec_tiled over int4-tiled routed experts,
G53H_MAT_I4T; the reference's --experts int4 mode at T = 1) and of the int4 tiling.

Bar: bit for bit. The routed experts are the reference's int4 (matmul_i4,
src/core/glm53f_ops.c:236-296: eight fp32 lanes per 64-column group, the pairwise double tree,
times the group's step, summed in double over the row), the shared expert FP8 (:185-228), the
router (:945-976) and the combine (:1329-1340). The outputs must equal the compiled
reference's golden output for config 2 (tests/golden/i4.npz), the five-launch row-major int4
path and the oracle, token for token."""
import ctypes as C
import os

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
import oracle_lib as O
from glm53h import DevBuf, check
from test_gpu_parity import same, say

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
G4 = np.load(os.path.join(HERE, "golden", "i4.npz"))


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


@pytest.fixture(scope="module")
def layers(L):
    sp = S.spec(2)
    say("building config-2 int4 layers: row-major and int4-tiled (288 experts each)")
    return S.DeviceLayer.build(sp, i4=True), S.DeviceLayer.build(sp, i4=True, tiled=True)


@pytest.mark.parametrize("rows,cols", [(2048, 4096), (4096, 2048), (8, 256), (24, 768)])
def test_i4_tile_device_equals_host(L, rows, cols):
    say("int4 tile", rows, cols)
    rng = np.random.default_rng(rows + cols)
    a = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    src, dst, back = DevBuf.from_array(a), DevBuf(a.nbytes), DevBuf(a.nbytes)
    check(L.g53h_tile_i4(dst.ptr, src.ptr, rows, cols, 0), "tile")
    check(L.g53h_tile_i4(back.ptr, dst.ptr, rows, cols, 1), "untile")
    want = np.zeros_like(a)
    assert L.g53h_tile_i4_host(want.ctypes.data, a.ctypes.data, rows, cols, 0) == 0
    assert np.array_equal(dst.download(np.uint8), want)
    assert np.array_equal(back.download(np.uint8), a)


def run(layer, x, given=None):
    sp = layer.sp
    xd, out, idx, w = DevBuf.from_array(x), DevBuf(sp.E * 4), DevBuf(sp.K * 4), DevBuf(sp.K * 4)
    if given is None:
        layer.forward(out, xd, 1, idx, w)
    else:
        gi, gw = DevBuf.from_array(given[0]), DevBuf.from_array(given[1])
        check(glm53h.lib().g53h_moe_routed_given(out.ptr, xd.ptr, 1, C.byref(layer.layer), gi.ptr, gw.ptr), "given")
    glm53h.sync()
    return out.download(np.float32), idx.download(np.int32), w.download(np.float32)


def test_i4tiled_decode_golden(L, layers):
    rm, tl = layers
    sp = tl.sp
    assert glm53h.lib().g53h_decode_errors() == 0
    say("int4-tiled decode, config 2, against the compiled reference's output")
    out, _, _ = run(tl, S.x_host(sp, 1, batch=0))
    assert same(out, G4["c2_out"])
    assert glm53h.lib().g53h_decode_errors() == 0


def test_i4tiled_decode_tokens(L, layers):
    rm, tl = layers
    sp = tl.sp
    x = S.x_host(sp, 6, batch=7)
    for t in range(6):
        say("int4-tiled decode token", t)
        got, ids, w = run(tl, x[t:t + 1])
        want_rm, ids_rm, w_rm = run(rm, x[t:t + 1])
        assert np.array_equal(ids, ids_rm) and same(w, w_rm) and same(got, want_rm), t
        if t < 2:
            qm = {int(e): rm.fetch_expert(int(e)) for e in ids}
            want, wi, _ = O.moe_i4(O.oracle(), x[t:t + 1], sp, rm.router_f32, rm.bias_f32, qm, rm.fetch_expert("shared"))
            assert np.array_equal(ids, wi[0]) and same(got, want[0]), t
            # the tiled copies hold the same levels
            qt = {int(e): tl.fetch_expert(int(e)) for e in ids[:2]}
            for e, mats in qt.items():
                for (wt, st), (wr, sr) in zip(mats, qm[e]):
                    assert np.array_equal(wt, wr) and np.array_equal(st, sr)
    assert glm53h.lib().g53h_decode_errors() == 0


def test_i4tiled_routing_given_and_batches_refused(L, layers):
    rm, tl = layers
    sp = tl.sp
    x = S.x_host(sp, 1, batch=9)
    got, ids, w = run(tl, x)
    say("int4-tiled decode with the routing given")
    got2, _, _ = run(tl, x, (ids.copy(), w.copy()))
    assert same(got, got2)
    x2 = DevBuf.from_array(S.x_host(sp, 2, batch=9))
    out2 = DevBuf(2 * sp.E * 4)
    assert glm53h.lib().g53h_moe(out2.ptr, x2.ptr, 2, C.byref(tl.layer), None, None) != 0
    glm53h.sync()
