"""bench.py - MI355X routed-expert MoE layer, BASELINE.json's metric on one GPU.

Workload: single-token decode of one MoE layer, hidden 4096,
moe_intermediate 2048, 288 routed experts all resident in HBM (FP8 E4M3, 128x128 fp32 block
scales, 25,171,968 B each), top-8 sigmoid router with correction bias, plus the shared expert.
A step is one layer call for one token (tokens cycle through 64 seeded inputs so routing
varies); inputs are resident in HBM when the timed region starts. Weights are seeded synthetic
(no checkpoint), generated in HBM.

Prints one JSON line: the layer time in microseconds (lower is better), achieved HBM GB/s,
the roofline of the dominant kernel (k_gateup) measured live with HIP events, and the
reference CPU expert path (compiled from the reference's sources, oracle/_ref) timed on this
host's cores on a bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps 400] [--warmup 50] [--no-cpu]
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
from glm53h import DevBuf, check  # noqa: E402

HBM_PEAK_GBPS = 8000.0      # MI355X HBM3E, vendor figure
NTOK = 64


def run_steps(L, layer, xs, outs, n, start=0):
    for i in range(n):
        t = (start + i) % NTOK
        check(L.g53h_moe(outs[t % 2].ptr, xs.ptr + t * layer.sp.E * 4, 1, C.byref(layer.layer), None, None),
              "g53h_moe")


def cpu_baseline(layer, x, idx_all, ncalls=20, warm=3):
    """The reference's glm53f_moe (oracle/_ref, built from the reference's own sources with its
    flags) on this host: config-2 decode of one token per call, experts in host RAM."""
    import oracle_lib as O
    if not O.have_ref():
        return None
    sp = layer.sp
    toks = list(range(4))
    need = sorted({int(e) for t in toks for e in idx_all[t]})
    mats = {e: layer.fetch_expert(e) for e in need}
    sh = layer.fetch_expert("shared")
    R = O.ref()
    times = []
    for i in range(warm + ncalls):
        t = toks[i % len(toks)]
        t0 = time.perf_counter()
        O.moe(R, x[t:t + 1], sp, layer.router_f32, layer.bias_f32, mats, sh)
        dt = time.perf_counter() - t0
        if i >= warm:
            times.append(dt)
    med = statistics.median(times)
    return {"value": round(med * 1e6, 1), "unit": "us/layer", "cores": int(os.environ.get("OMP_NUM_THREADS",
                                                                                      os.cpu_count())),
            "kind": "reference",
            "sample": f"reference glm53f_moe (src/core/glm53f_ops.c) compiled -O3 -mavx2 -mfma -fopenmp "
                      f"-ffp-contract=off, config-2 decode of 4 seeded tokens, {warm} warm-up + median of "
                      f"{ncalls} calls, experts in host RAM",
            "gbps": round(layer.algorithmic_bytes(sp.K) / med / 1e9, 2)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1:
        sys.exit("bench.py measures one GPU: this build has no multi-GPU path (expert-parallel "
                 "sharding is a design note only); run with --gpus 1")
    L = glm53h.init(0)
    sp = S.spec(2)
    layer = S.DeviceLayer.build(sp)
    x = S.x_host(sp, NTOK, batch=0)
    xs = DevBuf.from_array(x)
    outs = [DevBuf(sp.E * 4), DevBuf(sp.E * 4)]

    # routing of the sample tokens (for the algorithmic byte count and the CPU sample)
    idx = DevBuf(NTOK * sp.K * 4)
    w = DevBuf(NTOK * sp.K * 4)
    check(L.g53h_router(idx.ptr, w.ptr, xs.ptr, NTOK, layer.router.ptr, 1, layer.bias.ptr, sp.NE, sp.E, sp.K,
                        sp.norm_topk, C.c_float(sp.routed_scale), None), "router")
    idx_all = idx.download(np.int32).reshape(NTOK, sp.K)

    run_steps(L, layer, xs, outs, a.warmup)
    glm53h.sync()
    check(L.g53h_mark(), "mark")
    run_steps(L, layer, xs, outs, a.steps)
    check(L.g53h_mark(), "mark")
    ms = L.g53h_elapsed_ms()
    glm53h.sync()
    us_layer = ms * 1e3 / a.steps

    # per-kernel times (events after every kernel), separate run
    check(L.g53h_prof_enable(1), "prof")
    run_steps(L, layer, xs, outs, 200)
    tms = (C.c_float * 8)()
    cnt = (C.c_int * 8)()
    check(L.g53h_prof_collect(tms, cnt, 8), "collect")
    check(L.g53h_prof_enable(0), "prof")
    per = {name: (tms[i] / cnt[i] * 1e3 if cnt[i] else None) for i, name in
           [(1, "router_us"), (2, "gateup_us"), (3, "down_us"), (6, "combine_us"), (7, "fused_layer_us")]}
    errs = L.g53h_decode_errors()
    if errs:
        sys.exit(f"the decode kernel reported error flags {errs}")

    nslot = sp.K + 1
    mat_bytes = sp.E * sp.I + (sp.E // sp.br) * (sp.I // sp.bc) * 4     # codes + scales of one matrix
    gateup_bytes = nslot * 2 * mat_bytes + sp.E * 4                      # 9 experts' gate+up, x
    layer_bytes = layer.algorithmic_bytes(sp.K) + sp.E * 4 * 2           # + x in, out
    gbps = layer_bytes / (us_layer * 1e-6) / 1e9
    if per.get("fused_layer_us"):
        dom_name, dom_bytes, dom_us = "k_moe_decode<32,16> (whole layer, one launch)", layer_bytes, per["fused_layer_us"]
    else:
        dom_name, dom_bytes, dom_us = "k_gateup<32>", gateup_bytes, per["gateup_us"]
    dom_gbps = dom_bytes / (dom_us * 1e-6) / 1e9

    cpu = None if a.no_cpu else cpu_baseline(layer, x, idx_all)
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
                   "tokens_cycled": NTOK, "parallelism": "single GPU"},
        "hbm_GBps": round(gbps, 1),
        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "algorithmic_bytes_per_layer": layer_bytes,
        "kernels_us": {k: (round(v, 2) if v else v) for k, v in per.items()},
        "roofline": {"bound": "hbm", "kernel": dom_name, "achieved": round(dom_gbps, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(dom_gbps / HBM_PEAK_GBPS, 4),
                     "traffic": None, "bytes_per_launch": dom_bytes, "avg_launch_us": round(dom_us, 2)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
