"""GPU parity of the grouped path (T >= 2) on octet-tiled experts (G53H_MAT_TILED, the layout of
the HBM cache's slots at the released shapes): the grouped kernels read the tiled units in place
and lay the activation planes out in the same column order within every 128-column block.

Bar (the grouped path's stated tolerance, as tests/test_gpu_grouped.py): routing bit-exact, every
output within 1e-2 absolute + 2e-3 relative of the oracle or of the exact per-token GPU kernels
on the same weights in the row-major layout."""
import ctypes as C

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
import oracle_lib as O
from glm53h import DevBuf, check
from test_gpu_grouped import MID, oracle_out, run, say, within

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


@pytest.mark.parametrize("T,shared", [(33, True), (300, True), (64, False)])
def test_grouped_tiled_mid_shapes_vs_oracle(L, T, shared):
    sp = S.LayerSpec(**MID, shared=shared)
    layer = S.DeviceLayer.build(sp, tiled=True)
    x = S.x_host(sp, T, batch=3)
    say("tiled mid shapes T", T, "shared", shared)
    out, idx, w = run(layer, x, 1, "g53h_moe_grouped")
    want, wi, ww = oracle_out(layer, x, idx)
    assert np.array_equal(idx, wi) and np.array_equal(w.view(np.uint32), ww.view(np.uint32))
    within(out, want, f"tiled mid T={T} shared={shared}")


def test_grouped_tiled_config4_vs_exact(L):
    """BASELINE config 4 (2048 tokens) on the tiled layer, against the exact per-token kernels on
    the same seeded weights stored row-major, every token; the oracle on 3 tokens."""
    sp = S.spec(2)
    say("config 4: building the tiled and the row-major layer")
    lt = S.DeviceLayer.build(sp, tiled=True)
    lr = S.DeviceLayer.build(sp)
    T = 2048
    x = S.x_host(sp, T, batch=11)
    out, idx, w = run(lt, x, 1)
    ref, ri, rw = run(lr, x, 0)
    assert np.array_equal(idx, ri) and np.array_equal(w.view(np.uint32), rw.view(np.uint32))
    within(out, ref, "tiled config 4 vs exact GPU path")
    sel = [0, 1000, 2047]
    want, wi, _ = oracle_out(lt, x[sel], idx[sel])
    assert np.array_equal(idx[sel], wi)
    within(out[sel], want, "tiled config 4 vs oracle")
    say("the exact per-token kernels refuse tiled experts")
    prev = L.g53h_set_grouped(0)
    try:
        xd, o = DevBuf.from_array(x[:4]), DevBuf(4 * sp.E * 4)
        assert L.g53h_moe(o.ptr, xd.ptr, 4, C.byref(lt.layer), None, None) == -1
    finally:
        L.g53h_set_grouped(prev)


def test_dropin_prefill_through_tiled_cache(L):
    """The drop-in glm53f_moe at T = 64 on the released shapes through the HBM cache (octet-tiled
    slots, used in place by the grouped kernels) against the same experts served from host
    memory (row-major views, staged), and the oracle on 3 tokens."""
    from test_gpu_cache import PoolSrc, make_cfg, new_cache
    from test_gpu_parity import fmat
    sp = S.spec(2)
    NP = 12
    cf = make_cfg(sp)
    cf.n_layers = 1
    pool = [S.expert_host(sp, p) for p in range(NP)]
    W, B = S.router_host(sp), S.bias_host(sp)
    sh = S.expert_host(sp, "shared")
    T = 64
    x = np.ascontiguousarray(S.x_host(sp, T, batch=9), np.float32)

    def run_dropin(src):
        w = glm53h.Glm53fMoeW()
        w.gate, w.bias = W.ctypes.data, B.ctypes.data
        (gw, gs), (uw, us), (dw, ds) = sh
        w.sh_gate, w.sh_up = fmat(gw, gs, sp.I, sp.E, sp.br, sp.bc), fmat(uw, us, sp.I, sp.E, sp.br, sp.bc)
        w.sh_down = fmat(dw, ds, sp.E, sp.I, sp.br, sp.bc)
        w.src = C.pointer(src)
        out = np.zeros((T, sp.E), np.float32)
        L.glm53f_moe(out.ctypes.data, x.ctypes.data, C.byref(w), C.byref(cf), T, None)
        assert L.g53h_grouped_errors() == 0
        return out

    prev = L.g53h_set_grouped(1)
    st = glm53h.G53hStore()
    check(L.g53h_store_synth_init(C.byref(st), sp.E, sp.I, 2, sp.NE, NP, sp.seed, C.c_float(sp.expert_sigma)), "store")
    try:
        say("drop-in prefill, host-memory experts (row-major grouped pass)")
        want = run_dropin(PoolSrc(sp, pool).src)
        say("drop-in prefill through the tiled cache")
        c = new_cache(cf, st, 40, 0)
        try:
            got = run_dropin(c.src)
        finally:
            L.glm53f_cache_free(C.byref(c))
    finally:
        L.g53h_store_synth_free(C.byref(st))
        L.g53h_set_grouped(prev)
        L.glm53f_forget_host_weights()
    within(got, want, "tiled cache vs host experts")
    idx, _ = O.router(O.oracle(), x, sp, W, B)
    sel = [0, 31, 63]
    mats = {int(e): pool[int(e) % NP] for e in np.unique(idx[sel])}
    ref, _, _ = O.moe(O.oracle(), x[sel], sp, W, B, mats, sh)
    within(got[sel], ref, "tiled cache vs oracle")
