"""bench.py - MI355X routed-expert MoE layer, BASELINE.json's metric on one GPU.

Workload: single-token decode of one MoE layer, hidden 4096,
moe_intermediate 2048, 288 routed experts all resident in HBM (FP8 E4M3, 128x128 fp32 block
scales, 25,171,968 B each), top-8 sigmoid router with correction bias, plus the shared expert.
A step is one layer call for one token. Tokens cycle through 64 seeded inputs, so the routed
experts change from step to step. The router and the shared expert are held at 12 addresses
used in turn (12 x 27.5 MB, more than the 256 MB last-level cache), so no step reads them from
that cache either. Inputs are resident in HBM when the timed region starts. Weights are seeded
synthetic (no checkpoint), generated in HBM.

Prints one JSON line: the layer time in microseconds (lower is better), achieved HBM GB/s, the
roofline of the dominant kernel (k_dec_experts) measured live with HIP events on the library's
stream, and the reference CPU expert path (compiled from the reference's sources, oracle/_ref)
timed on this host's cores on a bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps 400] [--warmup 50] [--no-cpu] [--cpu-seconds 10]
       python bench.py --copy-calibration   (device-to-device copies of 256 MiB, for scaling
                                             rocprof's FETCH_SIZE / WRITE_SIZE counters)
"""
import argparse
import ctypes as C
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "glm-5.3-flash-in-c_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

import glm53h  # noqa: E402
import glm53h.synth as S  # noqa: E402
from glm53h import DevBuf, G53hExpert, G53hMoeLayer, check  # noqa: E402

HBM_PEAK_GBPS = 8000.0      # MI355X HBM3E, vendor figure
NTOK = 64
NCOPY = 12                  # router / shared-expert address copies used in turn


class Copies:
    """NCOPY layers that share the routed experts but hold the router and the shared expert at
    different addresses (same bytes, so routing and results are unchanged)."""

    def __init__(self, layer):
        sp, L = layer.sp, glm53h.lib()
        self.layers, self.keep = [], []
        sh = layer.experts[sp.NE]
        mats = (sh.gate, sh.up, sh.down)
        for c in range(NCOPY):
            if c == 0:
                self.layers.append(layer.layer)
                continue
            router = DevBuf(layer.router.nbytes)
            check(L.g53h_d2d(router.ptr, layer.router.ptr, layer.router.nbytes), "d2d")
            copies = []
            for m in mats:
                w = DevBuf(m.rows * m.cols)
                s = DevBuf(((m.rows + m.br - 1) // m.br) * m.scols * 4)
                check(L.g53h_d2d(w.ptr, m.w, w.nbytes), "d2d")
                check(L.g53h_d2d(s.ptr, m.s, s.nbytes), "d2d")
                copies.append((w, s, m))
                self.keep += [w, s]
            desc = G53hExpert(*[type(m)(w.ptr, s.ptr, m.rows, m.cols, m.br, m.bc, m.scols, 0)
                                for w, s, m in copies])
            dbuf = DevBuf.from_array(np.frombuffer(bytes(desc), np.uint8))
            self.keep += [router, dbuf]
            lay = G53hMoeLayer()
            C.memmove(C.byref(lay), C.byref(layer.layer), C.sizeof(G53hMoeLayer))
            lay.router, lay.shared = router.ptr, dbuf.ptr
            self.layers.append(lay)
        check(L.g53h_sync(), "sync")


def run_steps(L, cp, xs, outs, E, n, start=0):
    for i in range(n):
        s = start + i
        t = s % NTOK
        check(L.g53h_moe(outs[s % 2].ptr, xs.ptr + t * E * 4, 1, C.byref(cp.layers[s % NCOPY]), None, None),
              "g53h_moe")


def cpu_baseline(layer, x, idx_all, seconds):
    """The reference's glm53f_moe (oracle/_ref, built from the reference's own sources with its
    flags) on this host: config-2 decode of one token per call, experts in host RAM, for about
    `seconds` of CPU time after 3 warm-up calls."""
    import oracle_lib as O
    if not O.have_ref():
        return None
    sp = layer.sp
    toks = list(range(4))
    need = sorted({int(e) for t in toks for e in idx_all[t]})
    mats = {e: layer.fetch_expert(e) for e in need}
    sh = layer.fetch_expert("shared")
    R = O.ref()
    for i in range(3):
        O.moe(R, x[toks[i % 4]:toks[i % 4] + 1], sp, layer.router_f32, layer.bias_f32, mats, sh)
    times, t_end = [], time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 20:
        t = toks[len(times) % len(toks)]
        t0 = time.perf_counter()
        O.moe(R, x[t:t + 1], sp, layer.router_f32, layer.bias_f32, mats, sh)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count()))
    return {"value": round(med * 1e6, 1), "unit": "us/layer", "cores": threads, "kind": "reference",
            "sample": f"reference glm53f_moe (src/core/glm53f_ops.c) compiled -O3 -mavx2 -mfma -fopenmp "
                      f"-ffp-contract=off, OpenMP threads {threads}; config-2 decode of 4 seeded tokens cycled, "
                      f"3 warm-up + median of {len(times)} calls ({sum(times):.1f} s), experts in host RAM",
            "gbps": round(layer.algorithmic_bytes(sp.K) / med / 1e9, 2)}


def copy_calibration():
    L = glm53h.init(0)
    n = 256 << 20
    a, b = DevBuf(n), DevBuf(n)
    for _ in range(5):
        check(L.g53h_d2d(b.ptr, a.ptr, n), "d2d")
    glm53h.sync()
    print(json.dumps({"copy_calibration_bytes": n, "copies": 5}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--copy-calibration", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1:
        sys.exit("bench.py measures one GPU: this build has no multi-GPU path (expert-parallel "
                 "sharding is a design note only); run with --gpus 1")
    if a.copy_calibration:
        return copy_calibration()
    L = glm53h.init(0)
    sp = S.spec(2)
    layer = S.DeviceLayer.build(sp)
    cp = Copies(layer)
    x = S.x_host(sp, NTOK, batch=0)
    xs = DevBuf.from_array(x)
    outs = [DevBuf(sp.E * 4), DevBuf(sp.E * 4)]

    # routing of the sample tokens (for the CPU sample)
    idx = DevBuf(NTOK * sp.K * 4)
    w = DevBuf(NTOK * sp.K * 4)
    check(L.g53h_router(idx.ptr, w.ptr, xs.ptr, NTOK, layer.router.ptr, 1, layer.bias.ptr, sp.NE, sp.E, sp.K,
                        sp.norm_topk, C.c_float(sp.routed_scale), None), "router")
    idx_all = idx.download(np.int32).reshape(NTOK, sp.K)

    run_steps(L, cp, xs, outs, sp.E, a.warmup)
    glm53h.sync()
    check(L.g53h_mark(), "mark")
    run_steps(L, cp, xs, outs, sp.E, a.steps)
    check(L.g53h_mark(), "mark")
    ms = L.g53h_elapsed_ms()
    glm53h.sync()
    us_layer = ms * 1e3 / a.steps

    # per-kernel times: events after every launch on the library's stream, separate run
    check(L.g53h_prof_enable(1), "prof")
    nprof = min(a.steps, 200)
    run_steps(L, cp, xs, outs, sp.E, nprof)
    tms = (C.c_float * 8)()
    cnt = (C.c_int * 8)()
    check(L.g53h_prof_collect(tms, cnt, 8), "collect")
    check(L.g53h_prof_enable(0), "prof")
    per = {name: (tms[i] / cnt[i] * 1e3 if cnt[i] else None) for i, name in
           [(1, "k_dec_route_us"), (7, "k_dec_experts_us")]}
    errs = L.g53h_decode_errors()
    if errs:
        sys.exit(f"the decode kernels reported error flags {errs}")

    eb = sp.expert_bytes()
    router_bytes = sp.NE * sp.E * 2 + sp.NE * 4                           # bf16 router + bias
    layer_bytes = layer.algorithmic_bytes(sp.K) + sp.E * 4 * 2           # + x in, out
    gbps = layer_bytes / (us_layer * 1e-6) / 1e9
    dom_bytes = (sp.K + 1) * eb                                          # 8 routed + shared expert
    dom_us = per["k_dec_experts_us"]
    dom_gbps = dom_bytes / (dom_us * 1e-6) / 1e9

    cpu = None if a.no_cpu else cpu_baseline(layer, x, idx_all, a.cpu_seconds)
    traffic = None                      # HBM bytes per launch from the committed counter summary
    tp = os.path.join(ROOT, "profiles", "k_dec_experts_config2_traffic.json")
    if os.path.exists(tp):
        with open(tp) as f:
            traffic = json.load(f).get("traffic_bytes")
    line = {
        "metric": "moe_decode_layer_time",
        "value": round(us_layer, 2),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms / a.steps, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded FP8 E4M3 experts N(0,0.02) absmax-quantised per 128x128 block; bf16 x ~N(0,1))",
        "config": {"workload": "BASELINE config 2: single-token decode of one MoE layer, hidden 4096, "
                               "moe_inter 2048, 288 experts resident in HBM, top-8 + 1 shared",
                   "tokens_cycled": NTOK, "router_shared_copies": NCOPY, "parallelism": "single GPU"},
        "hbm_GBps": round(gbps, 1),
        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "algorithmic_bytes_per_layer": layer_bytes,
        "kernels_us": {k: (round(v, 2) if v else v) for k, v in per.items()},
        "roofline": {"bound": "hbm", "kernel": "k_dec_experts", "achieved": round(dom_gbps, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(dom_gbps / HBM_PEAK_GBPS, 4),
                     "traffic": traffic, "bytes_per_launch": dom_bytes, "avg_launch_us": round(dom_us, 2),
                     "router_kernel": {"kernel": "k_dec_route", "bytes_per_launch": router_bytes,
                                       "avg_launch_us": round(per["k_dec_route_us"], 2)}},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
