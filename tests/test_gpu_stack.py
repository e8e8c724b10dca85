"""Config 5 as a test: a stack of 8 routed-expert layers at the released shapes (hidden 4096,
inter 2048, 288 experts, top-8, shared expert) in single-token decode through the drop-in and
the HBM cache (src/cache/glm53f_cache.c:128-306 is the reference's), with the calibrated
Zipf(1.1) routing and correlated inputs of the bench and a budget of 40 slots for 2,304
experts, so reads, evictions and prefetch reads all happen. Every (layer, expert) key has its
own payload (the pinned store's codes come from a pool of 24, its block scales are the key's
own), so a slot handed back for the wrong key changes the output. Every output equals the
oracle's bit for bit, and equals the one from a cache large enough to never evict, without
prefetch (the cache decides what is resident when, never what a layer returns). The same run
with the drop-in's speculative layer turned off (route, fetch, then compute) returns the same
outputs (what the cache reads ahead, and when, depends on when copies are seen complete, in
the reference as here, so its counts may differ). With GLM53F_CACHE_MFMA set, the slots hold the
codes MFMA-tiled and the drop-in decodes on the FP8 matrix cores: the same stack's outputs are
within the path's tolerance (1e-2 abs + 2e-3 rel) of the bit-exact ones, speculative once every
expert is resident, and a three-token chunk through those slots is within it of the oracle."""
import ctypes as C
import os

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
import oracle_lib as O
from glm53h import check, zipf
from test_gpu_grouped import within
from test_gpu_parity import cfg_struct, fmat, same, say

pytestmark = pytest.mark.gpu
NL, STEPS, NP = 8, 4, 24


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


def test_stack_through_cache_with_misses(L):
    sps = [S.spec(3, layer=l) for l in range(NL)]
    sp = sps[0]
    c = dict(E=sp.E, I=sp.I, NE=sp.NE, K=sp.K, routed_scale=sp.routed_scale, norm_topk=sp.norm_topk,
             limit=sp.limit, br=sp.br, bc=sp.bc)
    cf = cfg_struct(c)
    cf.n_layers = NL
    W = [S.router_host(s_) for s_ in sps]
    B = [S.bias_host(s_) for s_ in sps]
    sh = S.expert_host(S.spec(2), "shared")
    rho = zipf.table(sp.NE, sp.K, sp.zipf_s)["rho"]
    rng = np.random.default_rng(3)
    bf = lambda v: (np.asarray(v, np.float32).view(np.uint32) + 0x8000 & 0xFFFF0000).view(np.float32)
    X = np.empty((STEPS, NL, sp.E), np.float32)
    cur = [bf(rng.standard_normal(sp.E)) for _ in range(NL)]
    for t in range(STEPS):
        for l in range(NL):
            cur[l] = bf(rho * cur[l] + np.sqrt(1 - rho * rho) * rng.standard_normal(sp.E))
            X[t, l] = cur[l]
    store = glm53h.G53hStore()
    say("building the pinned store of", NP, "experts")
    check(L.g53h_store_synth_init(C.byref(store), sp.E, sp.I, NL + 1, sp.NE, NP, sp.seed, C.c_float(sp.expert_sigma)),
          "store")
    check(L.g53h_store_synth_key_scales(C.byref(store)), "key scales")

    def shared_w(l, pf=0):
        w = glm53h.Glm53fMoeW()
        w.gate, w.bias = W[l].ctypes.data, B[l].ctypes.data
        (gw, gs), (uw, us), (dw, ds) = sh
        w.sh_gate = fmat(gw, gs, sp.I, sp.E, sp.br, sp.bc)
        w.sh_up = fmat(uw, us, sp.I, sp.E, sp.br, sp.bc)
        w.sh_down = fmat(dw, ds, sp.E, sp.I, sp.br, sp.bc)
        w.layer, w.prefetch_n = l, pf
        return w

    def run(slots, n_io, pf, passes=1, chunk=0):
        cache = glm53h.Glm53fCache()
        probe = glm53h.Glm53fCache()
        assert L.g53h_cache_init_store(C.byref(probe), C.byref(store), C.byref(cf), 1 << 30, 0, 0) == 0
        sb = probe.slot_bytes
        L.glm53f_cache_free(C.byref(probe))
        assert L.g53h_cache_init_store(C.byref(cache), C.byref(store), C.byref(cf), sb * slots, n_io, 0) == 0
        def one_pass():
            outs = np.zeros((STEPS, NL, sp.E), np.float32)
            for t in range(STEPS):
                for l in range(NL):
                    w = glm53h.Glm53fMoeW()
                    w.gate, w.bias = W[l].ctypes.data, B[l].ctypes.data
                    (gw, gs), (uw, us), (dw, ds) = sh
                    w.sh_gate = fmat(gw, gs, sp.I, sp.E, sp.br, sp.bc)
                    w.sh_up = fmat(uw, us, sp.I, sp.E, sp.br, sp.bc)
                    w.sh_down = fmat(dw, ds, sp.E, sp.I, sp.br, sp.bc)
                    w.src = C.pointer(cache.src)
                    w.layer, w.prefetch_n = l, pf
                    if l + 1 < NL:
                        w.next_gate, w.next_bias = W[l + 1].ctypes.data, B[l + 1].ctypes.data
                    o = np.zeros((1, sp.E), np.float32)
                    xt = np.ascontiguousarray(X[t, l:l + 1])
                    L.glm53f_moe(o.ctypes.data, xt.ctypes.data, C.byref(w), C.byref(cf), 1, None)
                    outs[t, l] = o[0]
            check(L.glm53f_cache_sync(C.byref(cache)), "sync")
            return outs

        try:
            runs = []
            for k in range(passes):
                if k:           # a fresh record of outcomes: the cold pass's misses no longer count
                    L.g53h_set_speculate(1)
                runs.append(one_pass())
            if chunk:           # a chunk of tokens on layer 0 through the same slots
                w = shared_w(0)
                w.src = C.pointer(cache.src)
                o = np.zeros((chunk, sp.E), np.float32)
                xt = np.ascontiguousarray(X[:chunk, 0])
                L.glm53f_moe(o.ctypes.data, xt.ctypes.data, C.byref(w), C.byref(cf), chunk, None)
                check(L.glm53f_cache_sync(C.byref(cache)), "sync")
                runs.append(o)
            stats = dict(kind=L.g53h_cache_slot_kind(C.byref(cache.src)), hits=cache.hits, misses=cache.misses, evictions=cache.evictions, bg_reads=cache.bg_reads,
                         bg_used=cache.bg_used, bytes=cache.bytes_read + cache.bg_bytes)
        finally:
            L.glm53f_cache_free(C.byref(cache))
        return (runs if passes > 1 or chunk else runs[0]), stats

    def counts():
        n = (C.c_int64 * 3)()
        L.g53h_speculate_counts(n)
        return list(n)

    try:
        counts()
        say("stack: 40 slots, prefetch 4 in flight, prefetch_n 6")
        got, st = run(40, 4, 6)
        sc = counts()
        say("stack stats", st, "layers speculative done / again / not", sc)
        assert sum(sc) == STEPS * NL
        prev = L.g53h_set_speculate(0)
        try:
            say("stack: the same without speculation")
            got0, st0 = run(40, 4, 6)
        finally:
            L.g53h_set_speculate(prev)
        assert counts()[:2] == [0, 0]
        say("without speculation", st0)
        assert np.array_equal(got.view(np.uint32), got0.view(np.uint32))
        assert st["misses"] > 0 and st["evictions"] > 0 and st["bg_reads"] > 0
        assert st["hits"] + st["misses"] == STEPS * NL * sp.K
        say("stack: 300 slots, no prefetch, the same tokens twice")
        L.g53h_set_speculate(1)
        (want, again), st2 = run(300, 0, 0, passes=2)
        sc2 = counts()
        say("layers speculative done / again / not", sc2)
        assert st2["evictions"] == 0
        # the second pass finds every expert resident: every layer finishes speculatively
        assert sc2[0] >= STEPS * NL and np.array_equal(want.view(np.uint32), again.view(np.uint32))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        # every output against the oracle, with each key's experts as the store hands them out
        def key_mats(l, e):
            q = glm53h.Glm53fExpertQ()
            assert store.view(C.cast(C.pointer(store), C.c_void_p), l, e, C.byref(q)) == 0
            out = []
            for m in (q.gate, q.up, q.down):
                nsc = ((m.rows + m.br - 1) // m.br) * m.scols
                w = np.frombuffer(C.string_at(m.w, m.rows * m.cols), np.uint8).copy()
                sc = np.frombuffer(C.string_at(m.s, nsc * 4), np.float32).copy()
                out.append((w, sc))
            return out

        distinct = set()
        for t in range(STEPS):
            for l in range(NL):
                idx, _ = O.router(O.oracle(), X[t, l:l + 1], sps[l], W[l], B[l])
                mats = {int(e): key_mats(l, int(e)) for e in idx[0]}
                for e, mm in mats.items():
                    distinct.add((l, e, float(mm[0][1][0])))
                o, oi, _ = O.moe(O.oracle(), X[t, l:l + 1], sps[l], W[l], B[l], mats, sh)
                assert np.array_equal(oi, idx) and same(got[t, l], o[0]), (t, l)
        say("oracle: all", STEPS * NL, "outputs equal;", len(distinct), "distinct (layer, expert) keys used")
        # no two keys share a first gate scale, so no two payloads are alike
        assert len({d[2] for d in distinct}) == len(distinct)
        assert st["kind"] == 1
        # the same stack through MFMA-tiled FP8 slots: the FP8 matrix-core decode
        os.environ["GLM53F_CACHE_MFMA"] = "1"
        try:
            say("stack: MFMA-tiled slots, 40 slots, prefetch 4 in flight, prefetch_n 6")
            gotm, stm = run(40, 4, 6)
            assert stm["kind"] == 2 and stm["misses"] > 0
            within(gotm.reshape(-1, sp.E), want.reshape(-1, sp.E), "MFMA-tiled cache with misses")
            say("stack: MFMA-tiled slots, 300 slots, the same tokens twice, then a 3-token chunk")
            counts()
            (m1, m2, mc), stm2 = run(300, 0, 0, passes=2, chunk=3)
            sc3 = counts()
            say("layers speculative done / again / not", sc3)
            assert sc3[0] >= STEPS * NL
            within(m2.reshape(-1, sp.E), want.reshape(-1, sp.E), "MFMA-tiled cache, speculative")
            idx, _ = O.router(O.oracle(), X[:3, 0], sps[0], W[0], B[0])
            mats = {int(e): key_mats(0, int(e)) for e in np.unique(idx)}
            o, oi, _ = O.moe(O.oracle(), X[:3, 0], sps[0], W[0], B[0], mats, sh)
            within(mc, o, "3-token chunk through MFMA-tiled slots")
        finally:
            del os.environ["GLM53F_CACHE_MFMA"]
    finally:
        L.g53h_store_synth_free(C.byref(store))
        L.glm53f_forget_host_weights()
