"""The drop-in's cached single-token decode (glm53f_moe through the HBM expert cache,
src/core/glm53f_ops.c:1144-1342 and src/cache/glm53f_cache.c:128-306 in the reference) on a small
stack whose experts all fit the cache: it prints the time per layer call, and is short enough to
run under a kernel tracer (a few hundred layer calls; the pinned store holds a pool of 24 experts
with per-key block scales, the shapes are the released ones: hidden 4096, inter 2048, 288 experts,
top-8, one shared expert).

    cd glm-5.3-flash-in-c_amd && python3 -m glm53h.stack_probe [--layers 8] [--steps 16]
"""
import argparse
import ctypes as C
import time

import numpy as np

import glm53h
from glm53h import check, zipf
import glm53h.synth as S


def _cfg(sp, n_layers):
    cf = glm53h.Glm53fCfg()
    cf.hidden, cf.moe_inter, cf.n_experts, cf.topk, cf.n_shared = sp.E, sp.I, sp.NE, sp.K, 1
    cf.routed_scale, cf.norm_topk, cf.swiglu_limit = sp.routed_scale, sp.norm_topk, sp.limit
    cf.fp8_block_r, cf.fp8_block_c = sp.br, sp.bc
    cf.n_layers = n_layers
    return cf


def _mat(w, s, rows, cols, br, bc):
    return glm53h.Glm53fMat(w.ctypes.data, s.ctypes.data, glm53h.GLM53F_WF8, rows, cols, br, bc, (cols + bc - 1) // bc)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--steps", type=int, default=16)
    ap.add_argument("--slots", type=int, default=1200, help="cache slots (25.2 MB each, 14.2 MB int4); the default holds every expert")
    ap.add_argument("--passes", type=int, default=3, help="timed passes over the steps, after two warm ones")
    ap.add_argument("--int4", type=int, default=0, choices=[0, 1, 2, 3],
                    help="the cache's int4 mode: 0 FP8 slots, 1 the reference's int4 slots, 2 int4-tiled slots, 3 int4 MFMA-tiled slots")
    a = ap.parse_args()
    L = glm53h.init(0)
    NL, STEPS = a.layers, a.steps
    sps = [S.spec(3, layer=l) for l in range(NL)]
    sp = sps[0]
    cf = _cfg(sp, NL)
    W = [S.router_host(s_) for s_ in sps]
    B = [S.bias_host(s_) for s_ in sps]
    (gw, gs), (uw, us), (dw, ds) = S.expert_host(S.spec(2), "shared")
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
    check(L.g53h_store_synth_init(C.byref(store), sp.E, sp.I, NL + 1, sp.NE, 24, sp.seed, C.c_float(sp.expert_sigma)),
          "store")
    check(L.g53h_store_synth_key_scales(C.byref(store)), "key scales")
    probe = glm53h.Glm53fCache()
    check(L.g53h_cache_init_store(C.byref(probe), C.byref(store), C.byref(cf), 1 << 30, 0, a.int4), "cache")
    sb = probe.slot_bytes
    L.glm53f_cache_free(C.byref(probe))
    cache = glm53h.Glm53fCache()
    check(L.g53h_cache_init_store(C.byref(cache), C.byref(store), C.byref(cf), sb * a.slots, 0, a.int4), "cache")
    ws = []
    for l in range(NL):
        w = glm53h.Glm53fMoeW()
        w.gate, w.bias = W[l].ctypes.data, B[l].ctypes.data
        w.sh_gate = _mat(gw, gs, sp.I, sp.E, sp.br, sp.bc)
        w.sh_up = _mat(uw, us, sp.I, sp.E, sp.br, sp.bc)
        w.sh_down = _mat(dw, ds, sp.E, sp.I, sp.br, sp.bc)
        w.src = C.pointer(cache.src)
        w.layer, w.prefetch_n = l, 6
        if l + 1 < NL:
            w.next_gate, w.next_bias = W[l + 1].ctypes.data, B[l + 1].ctypes.data
        ws.append(w)
    o = np.zeros((1, sp.E), np.float32)
    xs = [[np.ascontiguousarray(X[t, l:l + 1]) for l in range(NL)] for t in range(STEPS)]

    def one_pass():
        for t in range(STEPS):
            for l in range(NL):
                L.glm53f_moe(o.ctypes.data, xs[t][l].ctypes.data, C.byref(ws[l]), C.byref(cf), 1, None)

    try:
        one_pass()                                   # the reads land
        check(L.glm53f_cache_sync(C.byref(cache)), "cache sync")
        L.g53h_set_speculate(1)
        one_pass()
        n = (C.c_int64 * 3)()
        L.g53h_speculate_counts(n)
        for _ in range(a.passes):
            t0 = time.perf_counter()
            one_pass()
            dt = time.perf_counter() - t0
            print("us per layer call %.2f" % (dt * 1e6 / (STEPS * NL)), flush=True)
        L.g53h_speculate_counts(n)
        print("layers speculative and done / run again / not speculative:", list(n), flush=True)
    finally:
        L.glm53f_cache_free(C.byref(cache))
        L.g53h_store_synth_free(C.byref(store))


if __name__ == "__main__":
    main()
