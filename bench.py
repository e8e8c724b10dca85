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
roofline of the layer kernel (k_dec_layer) measured live with HIP events on the library's
stream, and the reference CPU expert path (compiled from the reference's sources, oracle/_ref)
timed on this host's cores on a bounded sample of the same workload.

Other BASELINE configs (one JSON line each, same contract), with --workload:
  3  batched decode: 64 tokens x top-8 over 288 experts with Zipf(1.1) popularity, one layer call
     of 64 tokens per step (the grouped FP8-MFMA path); metric us per 64-token layer call
  4  prefill: 2048 tokens, uniform routing, one layer call per step (grouped path); metric ms
     per layer, with TFLOP/s against the FP8 dense peak and GB/s against the HBM floor
  5  42-layer decode stack, 32 steps, through the drop-in glm53f_moe with the HBM expert cache
     (200 GB of slots) filled from pinned host memory and next-layer prefetch; metric us per
     layer, with hit rate and host-to-HBM GB/s

Usage: python bench.py [--gpus 1] [--steps 400] [--warmup 50] [--no-cpu] [--cpu-seconds 10]
       python bench.py --workload 3|4|5 [--steps K] [--warmup W] [--no-cpu]
       python bench.py --copy-calibration   (device-to-device copies of 256 MiB, for scaling
                                             rocprof's FETCH_SIZE / WRITE_SIZE counters)
"""
import argparse
import ctypes as C
import json
import os
import statistics
import subprocess
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
FP8_PEAK_TFLOPS = 5000.0    # MI355X dense FP8 matrix peak, vendor figure
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
            desc = G53hExpert(*[type(m)(w.ptr, s.ptr, m.rows, m.cols, m.br, m.bc, m.scols, m.flags)
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


def host_cpu():
    """The host the CPU baseline ran on: lscpu's model name, nproc (the CPUs this process may
    use) and the OpenMP threads the reference ran with."""
    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.lower().startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        nproc = int(subprocess.run(["nproc"], capture_output=True, text=True, timeout=10).stdout.strip())
    except (OSError, ValueError, subprocess.SubprocessError):
        nproc = len(os.sched_getaffinity(0))
    return {"lscpu_model": model, "nproc": nproc, "omp_threads": int(os.environ.get("OMP_NUM_THREADS", nproc))}


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
    moe = O.moe_i4 if layer.i4 else O.moe             # int4 layers: the reference's int4 experts
    for i in range(3):
        moe(R, x[toks[i % 4]:toks[i % 4] + 1], sp, layer.router_f32, layer.bias_f32, mats, sh)
    times, t_end = [], time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 20:
        t = toks[len(times) % len(toks)]
        t0 = time.perf_counter()
        moe(R, x[t:t + 1], sp, layer.router_f32, layer.bias_f32, mats, sh)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    threads = host_cpu()["omp_threads"]
    return {"value": round(med * 1e6, 1), "unit": "us/layer", "cores": threads, "host": host_cpu(), "kind": "reference",
            "sample": f"reference glm53f_moe (src/core/glm53f_ops.c) compiled -O3 -mavx2 -mfma -fopenmp "
                      f"-ffp-contract=off, OpenMP threads {threads}; config-2 decode of 4 seeded tokens cycled, "
                      f"3 warm-up + median of {len(times)} calls ({sum(times):.1f} s), experts in host RAM"
                      + (", routed experts int4 (GLM53F_WI4)" if layer.i4 else ""),
            "gbps": round(layer.algorithmic_bytes(sp.K) / med / 1e9, 2)}


def copy_calibration():
    L = glm53h.init(0)
    n = 256 << 20
    a, b = DevBuf(n), DevBuf(n)
    for _ in range(5):
        check(L.g53h_d2d(b.ptr, a.ptr, n), "d2d")
    glm53h.sync()
    print(json.dumps({"copy_calibration_bytes": n, "copies": 5}), flush=True)


def prof_run(L, fn, n, tags):
    """Per-kernel averages (us) over n calls of fn, from the library's HIP events."""
    check(L.g53h_prof_enable(1), "prof")
    for i in range(n):
        fn(i)
    tms = (C.c_float * 8)()
    cnt = (C.c_int * 8)()
    check(L.g53h_prof_collect(tms, cnt, 8), "collect")
    check(L.g53h_prof_enable(0), "prof")
    return {name: (round(tms[i] / cnt[i] * 1e3, 2) if cnt[i] else None) for i, name in tags}


def cpu_grouped(layer, x, idx, seconds):
    """The reference's glm53f_moe (oracle/_ref) on this host for the same token batch, experts in
    host RAM: one call of all T tokens per sample (the reference splits them into 64-token
    chunks itself), repeated for about `seconds`."""
    import oracle_lib as O
    if not O.have_ref():
        return None
    sp = layer.sp
    mats = {int(e): layer.fetch_expert(int(e)) for e in np.unique(idx)}
    sh = layer.fetch_expert("shared")
    R = O.ref()
    O.moe(R, x[:2], sp, layer.router_f32, layer.bias_f32, mats, sh)          # warm-up
    times, t_end = [], time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 1:
        t0 = time.perf_counter()
        O.moe(R, x, sp, layer.router_f32, layer.bias_f32, mats, sh)
        times.append(time.perf_counter() - t0)
    threads = host_cpu()["omp_threads"]
    return statistics.median(times), len(times), threads


def bench_grouped(a):
    """BASELINE configs 3 and 4 on the grouped path (g53h_moe with T tokens)."""
    L = glm53h.init(0)
    cfg = a.workload
    sp = S.spec(3 if cfg == 3 else 2)
    T = 64 if cfg == 3 else 2048
    steps = a.steps if a.steps != 400 else (200 if cfg == 3 else 30)
    warm = a.warmup if a.warmup != 50 else 5
    lay = "tiled" if a.layout == "mfma" else a.layout      # the grouped kernels read octet-tiled experts
    layer = S.DeviceLayer.build(sp, tiled=lay == "tiled")
    nb = 4
    xs = [S.x_host(sp, T, batch=b) for b in range(nb)]
    xd = [DevBuf.from_array(x) for x in xs]
    out = DevBuf(T * sp.E * 4)
    idx = DevBuf(T * sp.K * 4)
    uniq = []
    for b in range(nb):
        check(L.g53h_moe(out.ptr, xd[b].ptr, T, C.byref(layer.layer), idx.ptr, None), "g53h_moe")
        uniq.append(len(np.unique(idx.download(np.int32))))
    assert L.g53h_grouped_errors() == 0

    def step(i):
        check(L.g53h_moe(out.ptr, xd[i % nb].ptr, T, C.byref(layer.layer), None, None), "g53h_moe")

    for i in range(warm):
        step(i)
    glm53h.sync()
    check(L.g53h_mark(), "mark")
    for i in range(steps):
        step(i)
    check(L.g53h_mark(), "mark")
    ms = L.g53h_elapsed_ms() / steps
    glm53h.sync()
    per = prof_run(L, step, min(steps, 40), [(1, "router"), (5, "k_grp_plan+k_grp_xq"), (2, "k_grp_gateup"),
                                              (3, "k_grp_down"), (6, "k_grp_combine")])
    D = float(np.mean(uniq))
    eb = sp.expert_bytes()
    gu_bytes = (D + 1) * 2 * (sp.I * sp.E + (sp.I // 128) * (sp.E // 128) * 4)
    layer_bytes = (D + 1) * eb + sp.NE * sp.E * 2 + sp.NE * 4 + T * sp.E * 4 * 2
    flops = 2.0 * (T * sp.K + T) * 3 * sp.E * sp.I
    gbps = layer_bytes / (ms * 1e-3) / 1e9
    tflops = flops / (ms * 1e-3) / 1e12
    gu_gbps = gu_bytes / (per["k_grp_gateup"] * 1e-6) / 1e9
    cpu = None
    if not a.no_cpu:
        r = cpu_grouped(layer, xs[0], _routing(L, layer, xd[0], T), a.cpu_seconds)
        if r:
            med, n, threads = r
            cpu = {"value": round(med * (1e6 if cfg == 3 else 1e3), 1), "unit": "us/layer" if cfg == 3 else "ms/layer",
                   "cores": threads, "host": host_cpu(), "kind": "reference",
                   "sample": f"reference glm53f_moe (src/core/glm53f_ops.c, 64-token chunks) compiled -O3 -mavx2 "
                             f"-mfma -fopenmp -ffp-contract=off, OpenMP threads {threads}; the same {T}-token batch "
                             f"(batch 0), median of {n} call(s), experts in host RAM",
                   "tflops": round(flops / med / 1e12, 3)}
    name = "moe_batched_decode_layer_time" if cfg == 3 else "moe_prefill_layer_time"
    line = {
        "metric": name,
        "value": round(ms * 1e3, 2) if cfg == 3 else round(ms, 4),
        "unit": "us/layer" if cfg == 3 else "ms/layer",
        "n_gpus": 1, "steps": steps, "warmup": warm, "ms_per_step": round(ms, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32 accumulate, fp8 MFMA",
        "data": "synthetic (seeded FP8 E4M3 experts N(0,0.02) absmax-quantised per 128x128 block; bf16 x ~N(0,1))",
        "config": {"workload": (f"BASELINE config 3: batched decode, {T} tokens x top-8, Zipf(1.1) popularity"
                                if cfg == 3 else f"BASELINE config 4: prefill, {T} tokens, uniform routing, + shared"),
                   "tokens": T, "token_batches_cycled": nb, "unique_routed_experts": D,
                   "expert_layout": lay, "parallelism": "single GPU"},
        "tokens_per_s": round(T / (ms * 1e-3), 1),
        "tflops": round(tflops, 2),
        "fp8_peak_frac": round(tflops / FP8_PEAK_TFLOPS, 4),
        "hbm_GBps": round(gbps, 1),
        "hbm_floor_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "algorithmic_bytes_per_layer": int(layer_bytes),
        "kernels_us": per,
        "roofline": {"bound": "hbm", "kernel": "k_grp_gateup", "achieved": round(gu_gbps, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gu_gbps / HBM_PEAK_GBPS, 4), "traffic": _traffic(cfg),
                     "bytes_per_launch": int(gu_bytes), "avg_launch_us": per["k_grp_gateup"]},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def prefill_beside(L, layer, sp, steps=10, warm=3):
    """BASELINE config 4 (2048-token prefill, uniform routing) on the config-2 layer just timed
    (config 4 has config 2's layer), so the default line carries the prefill FP8 TFLOP/s that
    BASELINE's metric names. Two token batches cycled; the same figures as --workload 4."""
    T = 2048
    xd = [DevBuf.from_array(S.x_host(sp, T, batch=b)) for b in range(2)]
    out = DevBuf(T * sp.E * 4)
    idx = DevBuf(T * sp.K * 4)
    check(L.g53h_moe(out.ptr, xd[0].ptr, T, C.byref(layer.layer), idx.ptr, None), "g53h_moe")
    D = float(len(np.unique(idx.download(np.int32))))
    for i in range(warm):
        check(L.g53h_moe(out.ptr, xd[i % 2].ptr, T, C.byref(layer.layer), None, None), "g53h_moe")
    glm53h.sync()
    check(L.g53h_mark(), "mark")
    for i in range(steps):
        check(L.g53h_moe(out.ptr, xd[i % 2].ptr, T, C.byref(layer.layer), None, None), "g53h_moe")
    check(L.g53h_mark(), "mark")
    ms = L.g53h_elapsed_ms() / steps
    glm53h.sync()
    if L.g53h_grouped_errors():
        sys.exit("the grouped kernels reported error flags")
    flops = 2.0 * (T * sp.K + T) * 3 * sp.E * sp.I
    layer_bytes = (D + 1) * sp.expert_bytes() + sp.NE * sp.E * 2 + sp.NE * 4 + T * sp.E * 4 * 2
    tflops = flops / (ms * 1e-3) / 1e12
    return {"workload": "BASELINE config 4: prefill of 2048 tokens on the same layer, uniform routing, + shared",
            "steps": steps, "warmup": warm, "ms_per_layer": round(ms, 4), "tflops": round(tflops, 2),
            "fp8_peak_frac": round(tflops / FP8_PEAK_TFLOPS, 4),
            "hbm_floor_frac": round(layer_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
            "unique_routed_experts": D}


def batched_beside(L, layer, steps=100, warm=5):
    """BASELINE config 3 (64 tokens, Zipf(1.1) popularity) on the config-2 layer just timed: config
    3 is config 2 with the calibrated Zipf selection bias, so only the bias is swapped in. Four
    token batches cycled; the same figures as --workload 3."""
    sp3 = S.spec(3)
    T = 64
    bias = DevBuf.from_array(S.bias_host(sp3))
    l3 = G53hMoeLayer.from_buffer_copy(layer.layer)
    l3.bias = bias.ptr
    xd = [DevBuf.from_array(S.x_host(sp3, T, batch=b)) for b in range(4)]
    out = DevBuf(T * sp3.E * 4)
    idx = DevBuf(T * sp3.K * 4)
    uniq = []
    for b in range(4):
        check(L.g53h_moe(out.ptr, xd[b].ptr, T, C.byref(l3), idx.ptr, None), "g53h_moe")
        uniq.append(len(np.unique(idx.download(np.int32))))
    for i in range(warm):
        check(L.g53h_moe(out.ptr, xd[i % 4].ptr, T, C.byref(l3), None, None), "g53h_moe")
    glm53h.sync()
    check(L.g53h_mark(), "mark")
    for i in range(steps):
        check(L.g53h_moe(out.ptr, xd[i % 4].ptr, T, C.byref(l3), None, None), "g53h_moe")
    check(L.g53h_mark(), "mark")
    ms = L.g53h_elapsed_ms() / steps
    glm53h.sync()
    if L.g53h_grouped_errors():
        sys.exit("the grouped kernels reported error flags")
    D = float(np.mean(uniq))
    layer_bytes = (D + 1) * sp3.expert_bytes() + sp3.NE * sp3.E * 2 + sp3.NE * 4 + T * sp3.E * 4 * 2
    return {"workload": "BASELINE config 3: 64 tokens x top-8, Zipf(1.1) popularity (the calibrated bias), same layer",
            "steps": steps, "warmup": warm, "us_per_layer": round(ms * 1e3, 2),
            "hbm_floor_frac": round(layer_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
            "unique_routed_experts": D}


def _traffic(cfg):
    """HBM bytes per launch of the dominant kernel from the committed counter summary, if any."""
    tp = os.path.join(ROOT, "profiles", f"k_grp_gateup_config{cfg}_traffic.json")
    if not os.path.exists(tp):
        return None
    with open(tp) as f:
        return json.load(f).get("traffic_bytes")


def _routing(L, layer, xd, T):
    sp = layer.sp
    idx, w = DevBuf(T * sp.K * 4), DevBuf(T * sp.K * 4)
    check(L.g53h_router(idx.ptr, w.ptr, xd.ptr, T, layer.router.ptr, 1, layer.bias.ptr, sp.NE, sp.E, sp.K,
                        sp.norm_topk, C.c_float(sp.routed_scale), None), "router")
    return idx.download(np.int32).reshape(T, sp.K)


def cpu_stack_layer(sp, W, b, x, sh, seconds):
    """The reference's glm53f_moe for one layer of the stack (one token), experts already in host
    RAM (the reference's cache would read misses from storage; that is not timed)."""
    import oracle_lib as O
    if not O.have_ref():
        return None
    idx, _ = O.router(O.oracle(), x[None, :], sp, W, b)
    mats = {int(e): S.expert_host(sp, int(e)) for e in idx[0]}
    R = O.ref()
    xt = x[None, :]
    O.moe(R, xt, sp, W, b, mats, sh)
    times, t_end = [], time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 20:
        t0 = time.perf_counter()
        O.moe(R, xt, sp, W, b, mats, sh)
        times.append(time.perf_counter() - t0)
    threads = host_cpu()["omp_threads"]
    return {"value": round(statistics.median(times) * 1e6, 1), "unit": "us/layer", "cores": threads,
            "host": host_cpu(), "kind": "reference",
            "sample": f"reference glm53f_moe, one stack layer (layer 0, one token), experts in host RAM (no storage "
                      f"reads), OpenMP threads {threads}, median of {len(times)} calls"}


def route_dev(L, x, W, b, K):
    """Top-K indices [T][K] of the device router (bf16 router weights) for host x [T][E]."""
    T, E = x.shape
    NE = W.shape[0]
    gate = DevBuf.from_array((np.ascontiguousarray(W, np.float32).view(np.uint32) >> 16).astype(np.uint16))
    xd, bd = DevBuf.from_array(np.ascontiguousarray(x, np.float32)), DevBuf.from_array(np.ascontiguousarray(b))
    idx, wd, flag = DevBuf(T * K * 4), DevBuf(T * K * 4), DevBuf(4)
    flag.zero()
    check(L.g53h_router(idx.ptr, wd.ptr, xd.ptr, T, gate.ptr, 1, bd.ptr, NE, E, K, 1, C.c_float(2.5), flag.ptr),
          "router")
    return idx.download(np.int32).reshape(T, K)


def routing_stats(ids, ranks, NE, K):
    """(popularity exponent over ranks 2-200, token-to-token reuse) of routing ids [T][K] whose
    experts have popularity ranks ranks[e] (0-based)."""
    from glm53h import zipf
    freq = np.bincount(ranks[ids.ravel()], minlength=NE) / ids.shape[0]
    m = np.zeros((ids.shape[0], NE), bool)
    np.put_along_axis(m, ids, True, 1)
    return zipf.slope(freq), float((m[1:] & m[:-1]).sum() / (K * (ids.shape[0] - 1)))


def stack_routing(L, W, B, X, specs, rho):
    """The routing the run saw, measured on the device router: per-layer popularity ranks are
    the bias order. Reported for the run's own tokens (all layers pooled by rank) and for a
    2048-token continuation of layer 0's input chain (a sample long enough for the exponent)."""
    NE, K = specs[0].NE, specs[0].K
    NL = len(W)
    ranks = [np.argsort(np.argsort(-B[l], kind="stable"), kind="stable") for l in range(NL)]
    ids = [route_dev(L, np.ascontiguousarray(X[:, l]), W[l], B[l], K) for l in range(NL)]
    freq = np.zeros(NE)
    reuse_n = 0
    for l in range(NL):
        freq += np.bincount(ranks[l][ids[l].ravel()], minlength=NE)
        m = np.zeros((ids[l].shape[0], NE), bool)
        np.put_along_axis(m, ids[l], True, 1)
        reuse_n += (m[1:] & m[:-1]).sum()
    from glm53h import zipf
    run_slope = zipf.slope(freq / (NL * X.shape[0]))
    run_reuse = reuse_n / (NL * K * (X.shape[0] - 1))
    rng = np.random.default_rng(55)
    cur = X[-1, 0].astype(np.float64)
    long_x = np.empty((2048, X.shape[2]), np.float32)
    for t in range(2048):
        cur = rho * cur + np.sqrt(1 - rho * rho) * rng.standard_normal(X.shape[2])
        cur = (cur.astype(np.float32).view(np.uint32) + 0x8000 & 0xFFFF0000).view(np.float32).astype(np.float64)
        long_x[t] = cur
    s_long, r_long = routing_stats(route_dev(L, long_x, W[0], B[0], K), ranks[0], NE, K)
    return {"target": {"zipf_s": specs[0].zipf_s, "reuse": 0.70, "rho": rho},
            "run_tokens": {"tokens": int(NL * X.shape[0]), "zipf_slope": round(-run_slope, 3),
                           "reuse": round(float(run_reuse), 3)},
            "layer0_2048_tokens": {"zipf_slope": round(-s_long, 3), "reuse": round(r_long, 3)}}


def policy_eval(path, NE, K):
    """LRU (this library's cache policy) against the Belady bound on the run's own routing
    trace, at the reference's two cache sizes (docs/PERFORMANCE.md:301-306), when traced."""
    if not path:
        return None
    from glm53h import route_trace
    r = route_trace.evaluate(path, slots=(952, 1508), warm=20, topk=K, n_experts=NE)
    r["trace"] = os.path.basename(path)
    return r


def bench_stack(a):
    """a 42-layer stack of routed-expert layers (config-2 shapes) in single-
    token decode, 32 steps, each layer one glm53f_moe call (the drop-in, with the reference's
    hint protocol: own experts, then the next layer's router on this input, prefetch_n 6). The
    experts come through the HBM cache (200 GB of slots) from pinned host memory. Per-layer
    routers are seeded bf16; the selection bias is glm53h.zipf's calibrated curve (top-8
    popularity min(1, c r^-1.1)) over a per-layer permutation, and each layer's input follows
    x <- rho x + sqrt(1 - rho^2) z (bf16) with rho calibrated for 70% token-to-token reuse. Both
    are measured back on the device router and reported. The cache starts holding the most
    popular experts of every layer (what 200 GB holds), then warms up under the workload."""
    if a.route_trace:                                   # read by the drop-in at its first call
        if os.path.exists(a.route_trace):
            os.remove(a.route_trace)
        os.environ["GLM53F_ROUTE_TOP16"] = a.route_trace
    L = glm53h.init(0)
    NL, steps, warm = a.stack_layers, (a.steps if a.steps != 400 else 32), (a.warmup if a.warmup != 50 else 8)
    base = S.spec(3)
    E, I, NE, K = base.E, base.I, base.NE, base.K
    from glm53h import zipf
    rho, pf, n_io = zipf.table(NE, K, base.zipf_s)["rho"], a.prefetch, 4
    cf = glm53h.Glm53fCfg()
    cf.hidden, cf.n_layers, cf.n_experts, cf.topk, cf.n_shared, cf.moe_inter = E, NL, NE, K, 1, I
    cf.routed_scale, cf.norm_topk, cf.swiglu_limit = base.routed_scale, base.norm_topk, base.limit
    cf.fp8_block_r, cf.fp8_block_c = 128, 128
    print(f"[bench] config 5: building the pinned host store ({NE} experts)", file=sys.stderr, flush=True)
    st = glm53h.G53hStore()
    check(L.g53h_store_synth_init(C.byref(st), E, I, NL + 1, NE, NE, base.seed, C.c_float(base.expert_sigma)), "store")
    cache = glm53h.Glm53fCache()
    budget = 200 * 10 ** 9
    # --experts int4: the reference's int4 mode, the experts re-quantised as they are read, a decode
    # layer one launch. int4: the cache's mode 3 (int4 MFMA-tiled slots, the FP4 matrix-core decode) under the default
    # --layout mfma, mode 2 (int4-tiled slots, bit-exact) under --layout tiled
    i4mode = (3 if a.layout == "mfma" else 2) if a.experts == "int4" else 0
    # FP8: MFMA-tiled slots (the FP8 matrix-core decode) under the default --layout mfma, octet-tiled
    # ones (the bit-exact decode) under --layout tiled; the cache reads the switch at its init
    mt = a.experts == "fp8" and a.layout == "mfma"
    if mt:
        os.environ["GLM53F_CACHE_MFMA"] = "1"
    else:
        os.environ.pop("GLM53F_CACHE_MFMA", None)
    if L.g53h_cache_init_store(C.byref(cache), C.byref(st), C.byref(cf), budget, n_io, i4mode) != 0:
        sys.exit("glm53f_cache_init failed")
    specs = [S.spec(3, layer=l) for l in range(NL)]
    W = [S.router_host(s_) for s_ in specs]
    B = [S.bias_host(s_) for s_ in specs]
    sh = S.expert_host(base, "shared")
    per_layer = cache.nslot // NL
    print(f"[bench] config 5: filling {per_layer} x {NL} slots of {cache.nslot}", file=sys.stderr, flush=True)
    for l in range(NL):
        ranked = np.argsort(-B[l], kind="stable")[:per_layer].astype(np.int32)
        for c0 in range(0, len(ranked), 64):
            ids = np.ascontiguousarray(ranked[c0:c0 + 64])
            cache.src.getmany(C.byref(cache.src), l, ids.ctypes.data_as(C.POINTER(C.c_int)), len(ids))
    check(L.glm53f_cache_sync(C.byref(cache)), "cache sync")
    rng = np.random.default_rng(5)

    def bf16(v):
        return (np.asarray(v, np.float32).view(np.uint32) + 0x8000 & 0xFFFF0000).view(np.float32)

    # every input of the run, made before the timed region: x <- rho x + sqrt(1 - rho^2) z per layer
    X = np.empty((warm + steps, NL, E), np.float32)
    cur = [bf16(rng.standard_normal(E)) for _ in range(NL)]
    for s_ in range(warm + steps):
        for l in range(NL):
            cur[l] = bf16(rho * cur[l] + np.sqrt(1 - rho * rho) * rng.standard_normal(E))
            X[s_, l] = cur[l]
    xs = [X[0, l] for l in range(NL)]
    ws = []
    for l in range(NL):
        w = glm53h.Glm53fMoeW()
        w.gate, w.bias = W[l].ctypes.data, B[l].ctypes.data
        (gw, gs), (uw, us), (dw, ds) = sh
        w.sh_gate = glm53h.Glm53fMat(gw.ctypes.data, gs.ctypes.data, glm53h.GLM53F_WF8, I, E, 128, 128, E // 128)
        w.sh_up = glm53h.Glm53fMat(uw.ctypes.data, us.ctypes.data, glm53h.GLM53F_WF8, I, E, 128, 128, E // 128)
        w.sh_down = glm53h.Glm53fMat(dw.ctypes.data, ds.ctypes.data, glm53h.GLM53F_WF8, E, I, 128, 128, I // 128)
        w.src = C.pointer(cache.src)
        w.layer, w.prefetch_n = l, pf
        if l + 1 < NL:
            w.next_gate, w.next_bias = W[l + 1].ctypes.data, B[l + 1].ctypes.data
        ws.append(w)
    out = np.zeros((1, E), np.float32)
    fn = L.glm53f_moe

    xptr = [[X[s_, l].ctypes.data for l in range(NL)] for s_ in range(warm + steps)]
    wref = [C.byref(w_) for w_ in ws]
    cref, optr = C.byref(cf), out.ctypes.data

    def step(s_):
        for l in range(NL):
            fn(optr, xptr[s_][l], wref[l], cref, 1, None)

    print("[bench] config 5: warm-up", file=sys.stderr, flush=True)
    for s_ in range(warm):
        step(s_)
    check(L.glm53f_cache_sync(C.byref(cache)), "cache sync")
    L.glm53f_cache_reset_stats(C.byref(cache))
    spec = (C.c_int64 * 3)()
    L.g53h_speculate_counts(spec)
    hprof = (C.c_double * 16)()
    if hasattr(L, "g53h_host_prof"):             # a build with the drop-in's host timers
        L.g53h_host_prof.argtypes = [C.c_void_p]
        L.g53h_host_prof(hprof)
    glm53h.sync()
    t0 = time.perf_counter()
    for s_ in range(steps):
        step(warm + s_)
    glm53h.sync()
    dt = time.perf_counter() - t0
    L.g53h_speculate_counts(spec)
    ktrace = None
    if a.decode_trace:          # one more step with the decode kernel's timestamps, per layer call
        tb = DevBuf(1024 * 192 * 8)                       # up to 1024 workgroups
        spans, routed = [], []
        for l in range(NL):
            tb.zero()
            set_trace = L.g53h_set_mfma_decode_trace if (mt or i4mode == 3) else L.g53h_set_tiled_decode_trace
            set_trace(tb.ptr)
            fn(optr, xptr[warm + steps - 1][l], wref[l], cref, 1, None)
            set_trace(None)
            glm53h.sync()
            t = tb.download(np.uint64).reshape(-1, 192).astype(np.int64)
            t = t[t[:, 0] > 0]
            if len(t):
                end = t[:, :16].max(1)
                spans.append((end.max() - t[:, 0].min()) / 100.0)
                routed.append((np.median(t[t[:, 1] > 0, 1]) - t[:, 0].min()) / 100.0 if (t[:, 1] > 0).any() else -1)
        if spans:
            ktrace = {"layers": len(spans), "kernel_us_mean": round(float(np.mean(spans)), 2),
                      "kernel_us_min": round(float(np.min(spans)), 2), "kernel_us_max": round(float(np.max(spans)), 2),
                      "routing_done_us_median": round(float(np.median(routed)), 2)}
    if hasattr(L, "g53h_host_prof"):
        L.g53h_host_prof(hprof)
        print("[bench] host timers (us per layer call):", " ".join(f"{i}:{hprof[i]:.1f}" for i in range(16)),
              file=sys.stderr, flush=True)
    us_layer = dt * 1e6 / (steps * NL)
    hits, misses, bg_reads, bg_used = cache.hits, cache.misses, cache.bg_reads, cache.bg_used
    h2d = cache.bytes_read + cache.bg_bytes
    # the link's rate on its own: 16 expert copies from the pinned store into a slot-sized buffer
    q = glm53h.Glm53fExpertQ()
    st.view(C.cast(C.pointer(st), C.c_void_p), 0, 0, C.byref(q))
    dbuf = DevBuf(int(cache.slot_bytes))
    mats = [q.gate, q.up, q.down]
    t1 = time.perf_counter()
    for _ in range(16):
        for m in mats:
            check(L.g53h_h2d(dbuf.ptr, m.w, m.rows * m.cols), "h2d")
    link = 16 * sum(m.rows * m.cols for m in mats) / (time.perf_counter() - t1) / 1e9
    L.glm53f_cache_report(C.byref(cache), b"config 5")
    routing = stack_routing(L, W, B, X, specs, rho)
    nslot = cache.nslot
    L.glm53f_cache_free(C.byref(cache))
    L.g53h_store_synth_free(C.byref(st))
    eb = base.expert_bytes()
    line = {
        "metric": "moe_stack_decode_layer_time",
        "value": round(us_layer, 2),
        "unit": "us/layer",
        "n_gpus": 1, "steps": steps, "warmup": warm, "ms_per_step": round(dt * 1e3 / steps, 3),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded FP8 experts; per-layer bf16 routers with Zipf(1.1) bias; correlated bf16 inputs)",
        "config": {"workload": (f"BASELINE config 5: {NL}-layer decode stack" if NL == 42 else
                                f"config 5 diagnostic: {NL}-layer decode stack (BASELINE's is 42)") +
                               f", {steps} steps, HBM expert cache of 200 GB, the rest in pinned host memory, "
                               "next-layer prefetch",
                   "layers": NL, "slots": nslot,
                   "routed_experts": (("int4 (the reference's int4 mode, re-quantised as read; " +
                                       ("int4 MFMA-tiled slots, FP4 matrix cores, within the tolerance)" if i4mode == 3
                                        else "int4-tiled slots, bit-exact)")) if i4mode else
                                      "fp8 (MFMA-tiled slots, FP8 matrix cores, within the tolerance)" if mt else
                                      "fp8 (octet-tiled slots, bit-exact)"),
                   "prefetch_n": pf, "prefetch_reads_in_flight": n_io, "input_correlation": rho,
                   "parallelism": "single GPU"},
        "routing": routing,
        "policy_eval": policy_eval(a.route_trace, NE, K),
        "hit_rate": round(hits / max(hits + misses, 1), 4),
        "miss_rate": round(misses / max(hits + misses, 1), 4),
        "misses_per_token": round(misses / steps, 2),
        "requests": int(hits + misses), "misses": int(misses),
        "decode_kernel_trace": ktrace,
        "speculative_layers": {"done": int(spec[0]), "run_again": int(spec[1]), "not_speculative": int(spec[2])},
        "prefetch_reads": int(bg_reads), "prefetch_used": int(bg_used),
        "h2d_GB": round(h2d / 1e9, 3), "h2d_GBps_avg": round(h2d / dt / 1e9, 2), "h2d_link_GBps": round(link, 2),
        "hbm_GBps_experts": round(((K * base.expert_i4_bytes() + eb) if i4mode else (K + 1) * eb) /
                                  (us_layer * 1e-6) / 1e9, 1),
        # (the reference's FP8 layer on the CPU; not measured for the int4 run)
        "cpu_baseline": None if (a.no_cpu or i4mode) else cpu_stack_layer(base, W[0], B[0], X[0, 0], sh,
                                                                          a.cpu_seconds),
    }
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--no-prefill", action="store_true",
                    help="config 2: leave out the config-3 and config-4 figures measured beside the decode line")
    ap.add_argument("--workload", type=int, default=2, choices=[2, 3, 4, 5])
    ap.add_argument("--route-trace", default=None,
                    help="config 5: write the decode routing trace (GLM53F_ROUTE_TOP16 format) to this file and "
                         "report LRU vs Belady misses per token on it (the trace costs time: not for timing)")
    ap.add_argument("--prefetch", type=int, default=6,
                    help="workload 5: next-layer experts hinted per layer (the reference's --prefetch, "
                         "src/cli/glm53f_run.c:258,284; 0 hints nothing)")
    ap.add_argument("--stack-layers", type=int, default=42,
                    help="config 5: layers in the stack (42 is BASELINE's; fewer, e.g. 24, fit every expert in the "
                         "200 GB cache, which isolates the per-layer cost from host reads)")
    ap.add_argument("--decode-trace", action="store_true",
                    help="config 5: after the timed steps, one step with the one-launch decode's timestamps "
                         "(kernel span and routing time per layer call; diagnostic)")
    ap.add_argument("--layout", default="mfma", choices=["mfma", "tiled", "rowmajor"],
                    help="config 2: expert code layout in HBM: MFMA-tiled (k_dec_mfma, FP8 matrix cores, outputs "
                         "within the path's tolerance), octet-tiled (the cache's slots; k_dec_tiled, bit-exact) or "
                         "row-major (k_dec_layer, bit-exact); configs 3-4: tiled or rowmajor; config 5: the cache's "
                         "slots MFMA-tiled (k_dec_mfma, within the tolerance) or octet-tiled (k_dec_tiled, bit-exact)")
    ap.add_argument("--experts", default="fp8", choices=["fp8", "int4"],
                    help="config 2: routed experts as the checkpoint's FP8 (the metric) or re-quantised to the "
                         "reference's int4 format (its --experts int4 mode): one launch on the FP4 matrix cores over "
                         "int4 MFMA-tiled experts (--layout mfma, within the tolerance), one launch over int4-tiled "
                         "slots (--layout tiled, bit-exact), or with --layout rowmajor the five-launch row-wave "
                         "kernels; config 5: the cache's int4 "
                         "mode 3 with int4 MFMA-tiled slots (--layout tiled: mode 2, int4-tiled slots, bit-exact); "
                         "200 GB then holds every expert of 42 layers")
    a = ap.parse_args()
    if a.gpus != 1:
        sys.exit("bench.py measures one GPU: this build has no multi-GPU path (expert-parallel "
                 "sharding is a design note only); run with --gpus 1")
    if a.copy_calibration:
        return copy_calibration()
    if a.workload in (3, 4):
        return bench_grouped(a)
    if a.workload == 5:
        return bench_stack(a)
    L = glm53h.init(0)
    sp = S.spec(2)
    i4 = a.experts == "int4"
    i4m = i4 and a.layout == "mfma"                     # int4: one launch on the FP4 matrix cores
    i4t = i4 and a.layout == "tiled"                    # int4: one launch over int4-tiled slots
    i4 = i4 and a.layout == "rowmajor"                  # (rowmajor: the five-launch row kernels)
    mfma = a.layout == "mfma"
    tiled = (a.layout == "tiled" and not i4) or i4t
    kname = ("k_rows" if i4 else "k_dec_tiled_i4" if i4t else "k_dec_mfma_i4" if i4m else "k_dec_mfma" if mfma
             else "k_dec_tiled" if tiled else "k_dec_layer")
    layer = S.DeviceLayer.build(sp, tiled=tiled, i4=i4 or i4t or i4m, mfma=mfma)
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

    # per-kernel times. One launch per step (every path but the row-major int4 one): the timed
    # region's per-step time is that kernel's average duration. The row-major int4 path's several
    # kernels: events after every launch on the library's stream, in a separate run (the events
    # add a gap after each launch, so these sum to more than a step)
    if i4:
        check(L.g53h_prof_enable(1), "prof")
        nprof = min(a.steps, 200)
        run_steps(L, cp, xs, outs, sp.E, nprof)
        tms = (C.c_float * 8)()
        cnt = (C.c_int * 8)()
        check(L.g53h_prof_collect(tms, cnt, 8), "collect")
        check(L.g53h_prof_enable(0), "prof")
        tags = [(1, "router_us"), (4, "row_kernels_us"), (6, "combine_us")]
        per = {name: (tms[i] / cnt[i] * 1e3 if cnt[i] else None) for i, name in tags}
    else:
        per = {kname + "_us": us_layer}
    errs = L.g53h_decode_errors()
    if errs:
        sys.exit(f"the decode kernels reported error flags {errs}")

    eb = sp.expert_bytes()
    router_bytes = sp.NE * sp.E * 2 + sp.NE * 4                           # bf16 router + bias
    layer_bytes = layer.algorithmic_bytes(sp.K) + sp.E * 4 * 2           # + x in, out
    gbps = layer_bytes / (us_layer * 1e-6) / 1e9
    dom_bytes = (sp.K + 1) * eb + router_bytes                           # router, 8 routed + shared
    # the timed region launches exactly one kernel per step, back to back on one stream, so its
    # per-step time is the kernel's average duration (the per-kernel events of the separate
    # profiled run add a gap after every launch and are reported beside it)
    dom_us = us_layer
    if i4:
        # int4: the three row-wave launches (gate, up, down of 8 int4 experts + the FP8 shared
        # expert) with the SwiGLU between them, timed together by the profiled run's events
        dom_bytes = sp.K * sp.expert_i4_bytes() + eb
        dom_us = per["row_kernels_us"]
    elif i4t or i4m:
        # int4 in one launch: the router, 8 int4 experts and the FP8 shared expert
        dom_bytes = sp.K * sp.expert_i4_bytes() + eb + router_bytes
    dom_gbps = dom_bytes / (dom_us * 1e-6) / 1e9

    cpu = None if a.no_cpu else cpu_baseline(layer, x, idx_all, a.cpu_seconds)
    # the bit-exact decode kernel on the octet-tiled copy of the same layer, and the grouped
    # kernels' configs 3 and 4 (they read octet-tiled or row-major experts)
    exact, olayer = None, layer
    if mfma:
        olayer = S.DeviceLayer.build(sp, tiled=True, i4=i4m)
        ocp = Copies(olayer)
        run_steps(L, ocp, xs, outs, sp.E, a.warmup)
        glm53h.sync()
        check(L.g53h_mark(), "mark")
        run_steps(L, ocp, xs, outs, sp.E, a.steps)
        check(L.g53h_mark(), "mark")
        ex_us = L.g53h_elapsed_ms() * 1e3 / a.steps
        if L.g53h_decode_errors():
            sys.exit("the bit-exact decode kernel reported error flags")
        ex_bytes = ((sp.K * sp.expert_i4_bytes() + sp.expert_bytes()) if i4m else (sp.K + 1) * sp.expert_bytes())
        ex_gbps = (ex_bytes + sp.NE * sp.E * 2 + sp.NE * 4) / (ex_us * 1e-6) / 1e9
        exact = {"kernel": "k_dec_tiled_i4" if i4m else "k_dec_tiled", "parity": "bit-exact with the reference",
                 "steps": a.steps,
                 "us_per_layer": round(ex_us, 2), "achieved_GBps": round(ex_gbps, 1),
                 "hbm_peak_frac": round(ex_gbps / HBM_PEAK_GBPS, 4)}
        del ocp
    prefill = None if (i4 or i4t or i4m or a.no_prefill) else prefill_beside(L, olayer, sp)
    batched = None if (i4 or i4t or i4m or a.no_prefill) else batched_beside(L, olayer)
    traffic = None                      # HBM bytes per launch from the committed counter summary
    tp = os.path.join(ROOT, "profiles", f"{kname}_config2{'_int4' if i4 or i4t or i4m else ''}_traffic.json")
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
                   "tokens_cycled": NTOK, "router_shared_copies": NCOPY,
                   "expert_layout": ("int4 row-major" if i4 else "int4-tiled" if i4t else
                                     "int4 MFMA-tiled" if i4m else a.layout),
                   "routed_experts": a.experts,
                   "parity": ("routing bit-exact, outputs within 1e-2 abs + 2e-3 rel (FP4 matrix cores, int4 "
                              "levels exact)" if i4m else
                              "routing bit-exact, outputs within 1e-2 abs + 2e-3 rel (FP8 matrix cores)" if mfma
                              else "bit-exact with the reference"),
                   "parallelism": "single GPU"},
        "hbm_GBps": round(gbps, 1),
        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "algorithmic_bytes_per_layer": layer_bytes,
        ("kernels_us_event_bracketed" if i4 else "kernels_us"): {k: (round(v, 2) if v else v) for k, v in per.items()},
        "roofline": {"bound": "hbm", "kernel": "k_rows_gateup + k_rows_down" if i4 else kname,
                     "achieved": round(dom_gbps, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(dom_gbps / HBM_PEAK_GBPS, 4),
                     "traffic": traffic, "bytes_per_launch": dom_bytes, "avg_launch_us": round(dom_us, 2)},
        "cpu_baseline": cpu,
        "bit_exact_config2": exact,
        "batched_config3": batched,
        "prefill_config4": prefill,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
