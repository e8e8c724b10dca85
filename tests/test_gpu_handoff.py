"""The device-resident hand-off (the reference GPU backend's layer_on_dev,
src/gpu/glm53f_gpu.c:1020-1041, copies xn to the host, runs glm53f_moe_routed there and copies
the result back): the drop-in takes x and out in HBM directly, so a HIP trunk calls it on its
own buffers with no copy of either. The outputs must equal the host-pointer calls bit for bit,
for a chunk of tokens (host-memory expert source) and for single-token decode through the HBM
cache, and both must equal the oracle's glm53f_moe / glm53f_moe_routed (the CPU path the
reference's hand-off runs) on the same inputs, bit for bit."""
import ctypes as C

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
import oracle_lib as O
from glm53h import DevBuf, check
from test_gpu_parity import HostSrc, cfg_struct, fmat, same, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


def moe_w(sp, W, b, sh, src, layer=0):
    w = glm53h.Glm53fMoeW()
    w.gate, w.bias = W.ctypes.data, b.ctypes.data
    (gw, gs), (uw, us), (dw, ds) = sh
    w.sh_gate, w.sh_up = fmat(gw, gs, sp.I, sp.E, sp.br, sp.bc), fmat(uw, us, sp.I, sp.E, sp.br, sp.bc)
    w.sh_down = fmat(dw, ds, sp.E, sp.I, sp.br, sp.bc)
    w.src = C.pointer(src)
    w.layer = layer
    return w


def both_ways(L, w, cf, x, routed):
    """(host-pointer output, device-pointer output) of glm53f_moe(_routed)."""
    fn = L.glm53f_moe_routed if routed else L.glm53f_moe
    T, E = x.shape
    host = np.zeros_like(x)
    fn(host.ctypes.data, x.ctypes.data, C.byref(w), C.byref(cf), T, None)
    xd, od = DevBuf.from_array(x), DevBuf(x.nbytes)
    od.zero()
    fn(od.ptr, xd.ptr, C.byref(w), C.byref(cf), T, None)
    glm53h.sync()
    return host, od.download(np.float32).reshape(T, E)


def test_device_pointers_chunk_and_decode(L):
    sp = S.spec(1)
    cf = cfg_struct(dict(E=sp.E, I=sp.I, NE=sp.NE, K=sp.K, routed_scale=sp.routed_scale, norm_topk=sp.norm_topk,
                         limit=sp.limit, br=sp.br, bc=sp.bc))
    W, b = S.router_host(sp), S.bias_host(sp)
    ex = {e: S.expert_host(sp, e) for e in range(sp.NE)}
    sh = S.expert_host(sp, "shared")
    src = HostSrc(cf, ex)
    w = moe_w(sp, W, b, sh, src.src)
    for T in (1, 5, 70):
        x = np.ascontiguousarray(S.x_host(sp, T, batch=11), np.float32)
        for routed in (False, True):
            say("hand-off with device pointers, T", T, "routed only" if routed else "with shared")
            h, d = both_ways(L, w, cf, x, routed)
            assert same(h, d)
            want, _, _ = O.moe(O.oracle(), x, sp, W, b, ex, None if routed else sh)
            assert same(d, want), (T, routed)
    L.glm53f_forget_host_weights()


def test_device_pointers_cached_decode(L):
    """Config 2 through the HBM cache (octet-tiled slots, the one-launch decode)."""
    sp = S.spec(2)
    cf = cfg_struct(dict(E=sp.E, I=sp.I, NE=sp.NE, K=sp.K, routed_scale=sp.routed_scale, norm_topk=sp.norm_topk,
                         limit=sp.limit, br=sp.br, bc=sp.bc))
    cf.n_layers = 1
    W, b = S.router_host(sp), S.bias_host(sp)
    sh = S.expert_host(sp, "shared")
    store = glm53h.G53hStore()
    check(L.g53h_store_synth_init(C.byref(store), sp.E, sp.I, 2, sp.NE, 16, sp.seed, C.c_float(sp.expert_sigma)),
          "store")
    cache = glm53h.Glm53fCache()
    try:
        assert L.g53h_cache_init_store(C.byref(cache), C.byref(store), C.byref(cf), 40 * 25174016, 2, 0) == 0
        w = moe_w(sp, W, b, sh, cache.src)

        def key_mats(e):
            q = glm53h.Glm53fExpertQ()
            assert store.view(C.cast(C.pointer(store), C.c_void_p), 0, e, C.byref(q)) == 0
            return [(np.frombuffer(C.string_at(m.w, m.rows * m.cols), np.uint8).copy(),
                     np.frombuffer(C.string_at(m.s, ((m.rows + m.br - 1) // m.br) * m.scols * 4), np.float32).copy())
                    for m in (q.gate, q.up, q.down)]

        for t in range(3):
            x = np.ascontiguousarray(S.x_host(sp, 1, batch=30 + t), np.float32)
            idx, _ = O.router(O.oracle(), x, sp, W, b)
            mats = {int(e): key_mats(int(e)) for e in idx[0]}
            for routed in (False, True):
                say("cached decode with device pointers, token", t, "routed only" if routed else "with shared")
                h, d = both_ways(L, w, cf, x, routed)
                assert same(h, d)
                want, _, _ = O.moe(O.oracle(), x, sp, W, b, mats, None if routed else sh)
                assert same(d, want), (t, routed)
        assert L.g53h_decode_errors() == 0
    finally:
        L.glm53f_cache_free(C.byref(cache))
        L.g53h_store_synth_free(C.byref(store))
        L.glm53f_forget_host_weights()
