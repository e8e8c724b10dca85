"""GPU parity of the octet-tiled decode kernel (k_dec_tiled, T = 1) and the layout conversion.

Bar: bit-exact routing and outputs against the C oracle, which restates the reference's
arithmetic (src/core/glm53f_ops.c:185-228, 486-494, 945-976, 1329-1340), and bit-identical to
the row-major one-launch kernel on the same experts. The tiled layout only reorders where the
codes sit; the products, the block tree, the block order of the row sums and the combine are
the reference's."""
import ctypes as C

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
import oracle_lib as O
from glm53h import DevBuf, check
from test_gpu_parity import run_layer, same, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


def oracle_check(layer, x, out, idx, w, drop=()):
    sp = layer.sp
    mats = {int(e): layer.fetch_expert(int(e)) for e in idx[0] if int(e) not in drop}
    sh = layer.fetch_expert("shared") if sp.shared else None
    want, wi, ww = O.moe(O.oracle(), x, sp, layer.router_f32, layer.bias_f32, mats, sh)
    assert np.array_equal(idx, wi) and same(w, ww)
    assert same(out, want)


@pytest.mark.parametrize("rows,cols", [(2048, 4096), (4096, 2048), (8, 128), (24, 384)])
def test_tile_device_equals_host(L, rows, cols):
    say("tile", rows, cols)
    rng = np.random.default_rng(rows + cols)
    a = rng.integers(0, 256, rows * cols, dtype=np.uint8)
    src, dst, back = DevBuf.from_array(a), DevBuf(a.nbytes), DevBuf(a.nbytes)
    check(L.g53h_tile_f8(dst.ptr, src.ptr, rows, cols), "tile")
    check(L.g53h_untile_f8(back.ptr, dst.ptr, rows, cols), "untile")
    want = np.empty_like(a)
    assert L.g53h_tile_f8_host(want.ctypes.data, a.ctypes.data, rows, cols, 0) == 0
    assert np.array_equal(dst.download(np.uint8), want)
    assert np.array_equal(back.download(np.uint8), a)


@pytest.fixture(scope="module")
def layers(L):
    say("building config-2 layers, row-major and tiled")
    sp = S.spec(2)
    return S.DeviceLayer.build(sp), S.DeviceLayer.build(sp, tiled=True)


def test_tiled_decode_config2(L, layers):
    rm, tl = layers
    sp = tl.sp
    assert L.g53h_set_fused_decode(1) == 1
    for t in range(6):
        x = S.x_host(sp, 1, batch=40 + t)
        say("tiled decode config 2, token", t)
        out, idx, w = run_layer(tl, x, 1)
        assert L.g53h_decode_errors() == 0
        o2, i2, w2 = run_layer(rm, x, 1)
        assert L.g53h_decode_errors() == 0
        assert np.array_equal(idx, i2) and same(w, w2) and same(out, o2)
        if t < 2:
            oracle_check(tl, x, out, idx, w)


def test_tiled_decode_golden_router(L, layers):
    """The committed config-2 golden routing (compiled reference) through the tiled kernel."""
    import os
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))
    _, tl = layers
    sp = tl.sp
    x = S.x_host(sp, 64, batch=0)
    for t in (0, 17, 63):
        _, idx, w = run_layer(tl, x[t:t + 1], 1)
        assert np.array_equal(idx[0], gold["c2r_idx"][t])
        assert same(w[0], gold["c2r_w"][t])


@pytest.mark.parametrize("NE,K,shared,norm", [(512, 4, False, 1), (288, 15, True, 1), (640, 8, True, 0)])
def test_tiled_decode_other_layouts(L, NE, K, shared, norm):
    sp = S.spec(2, NE=NE, K=K, shared=shared, norm_topk=norm, seed=11)
    say("tiled decode layout NE", NE, "K", K, "shared", shared, "norm_topk", norm)
    layer = S.DeviceLayer.build(sp, tiled=True)
    for t in range(2):
        x = S.x_host(sp, 1, batch=20 + t)
        out, idx, w = run_layer(layer, x, 1)
        assert L.g53h_decode_errors() == 0
        oracle_check(layer, x, out, idx, w)
    del layer


def test_tiled_decode_absent_and_unusable_experts(L):
    """A routed expert without codes contributes zero (the reference's drop path); one that is
    not tiled, or has other blocks, is flagged (bit 8) and contributes zero too."""
    sp = S.spec(2, seed=12)
    layer = S.DeviceLayer.build(sp, tiled=True)
    x = S.x_host(sp, 1, batch=30)
    _, idx, _ = run_layer(layer, x, 1)
    gone, bad, rowmajor = int(idx[0][2]), int(idx[0][5]), int(idx[0][7])
    say("tiled decode with expert", gone, "absent,", bad, "unusable and", rowmajor, "row-major")
    descs = (glm53h.G53hExpert * (sp.NE + 1)).from_buffer_copy(bytes(layer.experts))
    descs[gone].gate.w = None
    descs[bad].up.bc = 64
    descs[rowmajor].down.flags = 0
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
                 wd.download(np.float32).reshape(1, sp.K), drop=(gone, bad, rowmajor))


def test_tiled_decode_ties(L, layers):
    """Equal choice values (identical router rows and biases): the reference's arg-max rounds
    take the lower expert index first (src/core/glm53f_ops.c:961-969, strict '>'). One tied
    group sits at the top of the ranking, one straddles the top-k boundary, so both the order
    of the slots and which of the tied experts make the cut are checked against the oracle."""
    _, base = layers
    sp = base.sp
    x = S.x_host(sp, 1, batch=77)
    _, idx0, _ = run_layer(base, x, 1)
    top, cut = int(idx0[0][0]), int(idx0[0][sp.K - 3])
    chosen = set(int(e) for e in idx0[0])
    free = [e for e in range(sp.NE) if e not in chosen]
    grp_top = [free[0], free[len(free) // 2], top]           # ties with the first choice
    grp_cut = [free[1], free[-1], cut]       # ties with the third-last: shifted two places by grp_top
    rf, bf = base.router_f32.copy(), base.bias_f32.copy()
    for grp in (grp_top, grp_cut):
        for e in grp[:-1]:
            rf[e] = rf[grp[-1]]
            bf[e] = bf[grp[-1]]
    router = DevBuf.from_array((rf.view(np.uint32) >> 16).astype(np.uint16))
    bias = DevBuf.from_array(bf)
    lay = glm53h.G53hMoeLayer.from_buffer_copy(bytes(base.layer))
    lay.router, lay.bias = router.ptr, bias.ptr
    xd = DevBuf.from_array(x)
    out, idd, wd = DevBuf(sp.E * 4), DevBuf(sp.K * 4), DevBuf(sp.K * 4)
    say("tiled decode with tied choices", grp_top, grp_cut)
    check(L.g53h_moe(out.ptr, xd.ptr, 1, C.byref(lay), idd.ptr, wd.ptr), "g53h_moe")
    glm53h.sync()
    assert L.g53h_decode_errors() == 0
    idx = idd.download(np.int32).reshape(1, sp.K)
    mats = {int(e): base.fetch_expert(int(e)) for e in idx[0]}
    want, wi, ww = O.moe(O.oracle(), x, sp, rf, bf, mats, base.fetch_expert("shared"))
    assert np.array_equal(idx, wi), (idx, wi)
    assert same(wd.download(np.float32).reshape(1, sp.K), ww)
    assert same(out.download(np.float32).reshape(1, sp.E), want)
    # the ties did shape the selection: the top group fills the first three slots in index order
    assert list(wi[0][:3]) == sorted(grp_top), wi[0]
    # the cut group now holds places K .. K + 2: only its lowest index is taken, in the last slot
    assert [int(e) for e in wi[0] if int(e) in grp_cut] == [min(grp_cut)] and int(wi[0][-1]) == min(grp_cut), wi[0]
