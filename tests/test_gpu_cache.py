"""GPU tests of the HBM expert cache (include/glm53f_cache.h) under the drop-in MoE layer.

The reference's contract (src/cache/glm53f_cache.h): the cache decides only what is resident
when; routing and arithmetic are unchanged, so outputs are bit-identical with any budget, with
prefetch on or off, and equal to the same layer served from host memory. A source whose get()
fails drops that expert (its contributions are zero, src/core/glm53f_ops.c:1261-1270). The
policy itself (LRU order, queue) is pinned against the reference's cache in
test_cache_policy.py."""
import ctypes as C

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
from glm53h import check
from test_gpu_parity import GOLD, HostSrc, cfg_struct, fmat, same, say

pytestmark = pytest.mark.gpu
N_MOE_LAYERS = 4


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


def make_cfg(sp):
    cf = cfg_struct(dict(E=sp.E, I=sp.I, NE=sp.NE, K=sp.K, routed_scale=sp.routed_scale, norm_topk=sp.norm_topk,
                         limit=sp.limit, br=sp.br, bc=sp.bc))
    cf.n_layers = N_MOE_LAYERS
    return cf


class Layers:
    """N_MOE_LAYERS MoE layers sharing config 1's router, bias and experts (expert e of every
    layer has the bytes of synthetic expert e), so the host-memory source and the synthetic
    store serve the same experts."""

    def __init__(self, sp):
        self.sp = sp
        self.W, self.b = S.router_host(sp), S.bias_host(sp)
        self.ex = {e: S.expert_host(sp, e) for e in range(sp.NE)}
        self.sh = S.expert_host(sp, "shared")

    def moe_w(self, src, layer, prefetch_n=0):
        sp, w = self.sp, glm53h.Glm53fMoeW()
        w.gate, w.bias = self.W.ctypes.data, self.b.ctypes.data
        (gw, gs), (uw, us), (dw, ds) = self.sh
        w.sh_gate, w.sh_up = fmat(gw, gs, sp.I, sp.E, sp.br, sp.bc), fmat(uw, us, sp.I, sp.E, sp.br, sp.bc)
        w.sh_down = fmat(dw, ds, sp.E, sp.I, sp.br, sp.bc)
        w.src = C.pointer(src)
        w.layer = layer
        w.prefetch_n = prefetch_n
        if prefetch_n and layer + 1 < N_MOE_LAYERS:
            w.next_gate, w.next_bias = self.W.ctypes.data, self.b.ctypes.data
        return w

    def run(self, src, cf, x, prefetch_n=0):
        """Every token through every layer, one decode call each; outputs [steps][layers][E]."""
        outs = []
        for t in range(x.shape[0]):
            per = []
            for layer in range(N_MOE_LAYERS):
                w = self.moe_w(src, layer, prefetch_n)
                xt = np.ascontiguousarray(x[t:t + 1], np.float32)
                out = np.zeros((1, self.sp.E), np.float32)
                glm53h.lib().glm53f_moe(out.ctypes.data, xt.ctypes.data, C.byref(w), C.byref(cf), 1, None)
                per.append(out[0])
            outs.append(per)
        return np.asarray(outs)


def new_cache(cf, st, slots, n_io):
    c = glm53h.Glm53fCache()
    L = glm53h.lib()
    assert L.g53h_cache_init_store(C.byref(c), C.byref(st), C.byref(cf), 0, 0, 0) == -1   # no slot fits
    probe = glm53h.Glm53fCache()
    assert L.g53h_cache_init_store(C.byref(probe), C.byref(st), C.byref(cf), 1 << 30, 0, 0) == 0
    budget = probe.slot_bytes * slots
    L.glm53f_cache_free(C.byref(probe))
    assert L.g53h_cache_init_store(C.byref(c), C.byref(st), C.byref(cf), budget, n_io, 0) == 0
    assert c.nslot == slots and L.g53h_cache_is(C.byref(c.src)) == 1
    return c


def test_cache_outputs_bit_identical(L):
    sp = S.spec(1)
    cf = make_cfg(sp)
    ly = Layers(sp)
    x = S.x_host(sp, 6, batch=2)
    say("cache: host-memory source (reference outputs)")
    want = ly.run(HostSrc(cf, ly.ex).src, cf, x)
    st = glm53h.G53hStore()
    check(L.g53h_store_synth_init(C.byref(st), sp.E, sp.I, N_MOE_LAYERS + 1, sp.NE, sp.NE, sp.seed,
                                  C.c_float(sp.expert_sigma)), "store")
    try:
        for slots, n_io, pf in [(sp.K + 1, 0, 0), (sp.K + 1, 2, 6), (12, 4, 6), (80, 2, 6), (80, 0, 0)]:
            say("cache: slots", slots, "prefetch reads in flight", n_io, "prefetch_n", pf)
            c = new_cache(cf, st, slots, n_io)
            try:
                got = ly.run(c.src, cf, x, prefetch_n=pf)
                check(L.glm53f_cache_sync(C.byref(c)), "sync")
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
                # one get per routed expert of every token and layer (top-k experts are distinct)
                assert c.hits + c.misses == x.shape[0] * N_MOE_LAYERS * sp.K
                assert c.bytes_read == (c.misses + c.prefetch_reads) * sp.expert_bytes()
                assert c.bg_bytes == c.bg_reads * sp.expert_bytes()
                if n_io:
                    assert c.bg_reads > 0 and c.bg_used > 0
                L.glm53f_cache_report(C.byref(c), b"test")
                if slots >= N_MOE_LAYERS * sp.NE:        # everything fits: a second pass only hits
                    L.glm53f_cache_reset_stats(C.byref(c))
                    again = ly.run(c.src, cf, x[:2], prefetch_n=pf)
                    assert np.array_equal(again.view(np.uint32), want[:2].view(np.uint32))
                    assert c.misses == 0 and c.hits == 2 * N_MOE_LAYERS * sp.K and c.bg_reads == 0
            finally:
                L.glm53f_cache_free(C.byref(c))
    finally:
        L.g53h_store_synth_free(C.byref(st))


class PyStore:
    """A G53hStore over host numpy arrays (pageable memory), failing for the dropped experts and
    counting view/done calls."""

    def __init__(self, sp, ex, drop=()):
        self.sp, self.ex, self.drop = sp, ex, set(drop)
        self.views, self.dones = 0, 0
        self.st = glm53h.G53hStore()
        self._v = glm53h.VIEW_FN(self.view)
        self._d = glm53h.DONE_FN(self.done)
        self.st.view, self.st.done = self._v, self._d

    def view(self, stp, layer, e, q):
        if e in self.drop:
            return -1
        self.views += 1
        sp = self.sp
        (gw, gs), (uw, us), (dw, ds) = self.ex[e]
        q[0].gate, q[0].up = fmat(gw, gs, sp.I, sp.E, sp.br, sp.bc), fmat(uw, us, sp.I, sp.E, sp.br, sp.bc)
        q[0].down = fmat(dw, ds, sp.E, sp.I, sp.br, sp.bc)
        return 0

    def done(self, stp, layer, e):
        self.dones += 1


def test_cache_drop_path_and_store_protocol(L):
    """A store that cannot read experts 3 and 7: the layer equals the reference's output with
    those experts dropped (golden, from the compiled reference), and every view is handed back
    with done() once its copy has landed."""
    sp = S.spec(1)
    cf = make_cfg(sp)
    ly = Layers(sp)
    store = PyStore(sp, ly.ex, drop=(3, 7))
    c = new_cache(cf, store.st, sp.K + 2, 0)
    try:
        w = ly.moe_w(c.src, 0)
        xb = np.ascontiguousarray(S.x_host(sp, 5, batch=1), np.float32)
        out = np.zeros((5, sp.E), np.float32)
        drops0 = C.c_long.in_dll(L, "glm53f_expert_drops").value
        say("cache: drop path, T=5")
        L.glm53f_moe(out.ctypes.data, xb.ctypes.data, C.byref(w), C.byref(cf), 5, None)
        assert same(out, GOLD["c1d_out"])
        assert C.c_long.in_dll(L, "glm53f_expert_drops").value > drops0
        check(L.glm53f_cache_sync(C.byref(c)), "sync")
        assert store.views > 0 and store.dones == store.views
    finally:
        L.glm53f_cache_free(C.byref(c))


def test_cache_rejects_empty_index_and_tiny_budgets(L):
    sp = S.spec(1)
    cf = make_cfg(sp)
    ly = Layers(sp)
    store = PyStore(sp, ly.ex)
    c = glm53h.Glm53fCache()
    ckpt = glm53h.Glm53fSt()
    assert L.glm53f_cache_init(C.byref(c), C.byref(ckpt), C.byref(cf), 1 << 30, 0, 1) == -1   # no tensors
    probe = glm53h.Glm53fCache()
    assert L.g53h_cache_init_store(C.byref(probe), C.byref(store.st), C.byref(cf), 1 << 30, 0, 0) == 0
    sb = probe.slot_bytes
    L.glm53f_cache_free(C.byref(probe))
    assert L.g53h_cache_init_store(C.byref(c), C.byref(store.st), C.byref(cf), sb * sp.K, 0, 0) == -1   # < topk+1


class PoolSrc:
    """A host-memory Glm53fExpertSrc serving the synthetic store's bytes: expert (L, e) is
    synthetic expert (L * n_experts + e) % n_pool."""

    def __init__(self, sp, pool):
        self.sp, self.pool = sp, pool
        self.src = glm53h.Glm53fExpertSrc()
        self._get = glm53h.GET_FN(self.get)
        self._rel = glm53h.RELEASE_FN(lambda *a: None)
        self.src.get, self.src.release = self._get, self._rel

    def get(self, selfp, layer, e, q):
        sp = self.sp
        (gw, gs), (uw, us), (dw, ds) = self.pool[(layer * sp.NE + e) % len(self.pool)]
        q[0].gate, q[0].up = fmat(gw, gs, sp.I, sp.E, sp.br, sp.bc), fmat(uw, us, sp.I, sp.E, sp.br, sp.bc)
        q[0].down = fmat(dw, ds, sp.E, sp.I, sp.br, sp.bc)
        return 0


def test_cache_config2_decode_through_fused_kernels(L):
    """Released shapes: two layers, four tokens each, through the cache (the drop-in's cached
    single-token path: one read-back of routing and prediction, the fused decode kernels on
    cache slots), bit-identical to the same experts served from host memory (the drop-in's
    general path)."""
    sp = S.spec(2)
    NP = 12
    cf = make_cfg(sp)
    cf.n_layers = 2
    pool = [S.expert_host(sp, p) for p in range(NP)]
    W = [S.router_host(S.spec(2, layer=l)) for l in range(2)]
    B = [S.bias_host(S.spec(2, layer=l)) for l in range(2)]
    sh = S.expert_host(sp, "shared")
    x = S.x_host(sp, 4, batch=7)

    def run(src, pf):
        outs = []
        for t in range(4):
            for l in range(2):
                w = glm53h.Glm53fMoeW()
                w.gate, w.bias = W[l].ctypes.data, B[l].ctypes.data
                (gw, gs), (uw, us), (dw, ds) = sh
                w.sh_gate = fmat(gw, gs, sp.I, sp.E, sp.br, sp.bc)
                w.sh_up = fmat(uw, us, sp.I, sp.E, sp.br, sp.bc)
                w.sh_down = fmat(dw, ds, sp.E, sp.I, sp.br, sp.bc)
                w.src = C.pointer(src)
                w.layer, w.prefetch_n = l, pf
                if pf and l == 0:
                    w.next_gate, w.next_bias = W[1].ctypes.data, B[1].ctypes.data
                out = np.zeros((1, sp.E), np.float32)
                xt = np.ascontiguousarray(x[t:t + 1])
                L.glm53f_moe(out.ctypes.data, xt.ctypes.data, C.byref(w), C.byref(cf), 1, None)
                outs.append(out[0])
        return np.asarray(outs)

    say("config 2 through host memory (general path)")
    host = PoolSrc(sp, pool)
    want = run(host.src, 0)
    st = glm53h.G53hStore()
    check(L.g53h_store_synth_init(C.byref(st), sp.E, sp.I, 3, sp.NE, NP, sp.seed, C.c_float(sp.expert_sigma)), "store")
    try:
        for slots, n_io, pf in [(sp.K + 1, 0, 0), (12, 2, 6)]:
            say("config 2 through the cache: slots", slots, "prefetch", n_io, pf)
            c = new_cache(cf, st, slots, n_io)
            try:
                got = run(c.src, pf)
                assert L.g53h_decode_errors() == 0
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
                assert c.hits + c.misses == 4 * 2 * sp.K
            finally:
                L.glm53f_cache_free(C.byref(c))
    finally:
        L.g53h_store_synth_free(C.byref(st))
