"""Cache policy evaluation on decode routing traces (the reference's GLM53F_ROUTE_TOP16 format,
src/core/glm53f_ops.c:1044-1080: one line per decode MoE layer, the layer, then the 16 best
candidates in selection order as id:score; the first top-k are the experts the layer used).
The drop-in writes the same lines from the device router when GLM53F_ROUTE_TOP16 names a file.

    python -m glm53h.route_trace TRACE [--slots 952 1508] [--warm 20] [--topk 8] [--experts 288]

Replays the used experts, in order, through
  lru     this library's expert cache policy (g53h_lru_trace: the HBM cache's own bookkeeping,
          pinned against the reference cache in tests/test_cache_policy.py): per layer-step a
          get of every used expert, then their release;
  belady  the clairvoyant bound (evict the resident expert whose next use is farthest away,
          Belady 1966), over the same access sequence;
and reports misses per token after the warm-up tokens (a token starts where the layer number
does not increase), the quantity of the reference's own table (docs/PERFORMANCE.md:301-306:
LRU 161.8 vs Belady 95.0 at 952 slots, 129.6 vs 71.1 at 1508, on its model's trace)."""
from __future__ import annotations

import argparse
import ctypes as C
import heapq
import json

import numpy as np


def load(path, topk=8):
    """[(layer, [(id, score)...])] from a trace file."""
    steps = []
    with open(path) as f:
        for line in f:
            p = line.split()
            if len(p) < 1 + topk:
                continue
            cand = []
            for t in p[1:]:
                a, b = t.split(":")
                cand.append((int(a), float(b)))
            steps.append((int(p[0]), cand))
    return steps


def tokens_of(steps):
    """Steps grouped into tokens: a new token starts when the layer number does not increase."""
    toks, cur, last = [], [], None
    for layer, cand in steps:
        if last is not None and layer <= last:
            toks.append(cur)
            cur = []
        cur.append((layer, cand))
        last = layer
    if cur:
        toks.append(cur)
    return toks


def accesses(toks, topk, n_experts):
    """(keys [n], token index of each access [n]) with key = layer * n_experts + expert."""
    keys, tix = [], []
    for ti, tok in enumerate(toks):
        for layer, cand in tok:
            for e, _ in cand[:topk]:
                keys.append(layer * n_experts + e)
                tix.append(ti)
    return np.asarray(keys, np.int64), np.asarray(tix, np.int64)


def lru_misses(toks, slots, warm, topk, n_experts, lib=None):
    """Misses per measured token through g53h_lru_trace (get every used expert of a step,
    then release them)."""
    if lib is None:
        from . import lib as _lib
        lib = _lib()
    n_layers = 1 + max(layer for tok in toks for layer, _ in tok)
    ops, marks = [], []
    for ti, tok in enumerate(toks):
        for layer, cand in tok:
            ids = [e for e, _ in cand[:topk]]
            for e in ids:
                ops += [1, layer, e]
                marks.append(ti)
            for e in ids:
                ops += [2, layer, e]
    ops = np.asarray(ops, np.int32)
    out = np.zeros(3 * len(marks) + 16, np.int32)
    stats = (C.c_longlong * 6)()
    n = lib.g53h_lru_trace(n_layers, n_experts, slots, ops.ctypes.data, len(ops), out.ctypes.data, len(out), stats)
    if n < 0:
        raise RuntimeError("g53h_lru_trace failed")
    res = out[:3 * len(marks)].reshape(-1, 3)
    if np.any(res[:, 0] != 0):
        raise RuntimeError("a get failed (fewer slots than one step holds)")
    marks = np.asarray(marks)
    miss = (res[:, 1] == 0) & (marks >= warm)
    return miss.sum() / max(len(toks) - warm, 1)


def lru_misses_py(keys, tix, slots, warm, n_tokens):
    """Plain LRU over the access sequence (no pins): a cross-check of the library's replay."""
    from collections import OrderedDict
    cache, misses = OrderedDict(), 0
    for k, t in zip(keys.tolist(), tix.tolist()):
        if k in cache:
            cache.move_to_end(k)
            continue
        misses += t >= warm
        cache[k] = 1
        if len(cache) > slots:
            cache.popitem(last=False)
    return misses / max(n_tokens - warm, 1)


def belady_misses(keys, tix, slots, warm, n_tokens):
    """Misses per measured token of the clairvoyant policy: on a miss with a full cache, evict
    the resident key whose next use is farthest (never used again counts as infinitely far).
    A max-heap of (next use, key) with stale entries skipped."""
    n = len(keys)
    nxt = np.full(n, n + 1, np.int64)
    last = {}
    for i in range(n - 1, -1, -1):
        k = int(keys[i])
        nxt[i] = last.get(k, n + 1 + i)            # distinct "never" positions keep keys apart
        last[k] = i
    resident = {}                                   # key -> its next use
    heap = []
    misses = 0
    for i in range(n):
        k = int(keys[i])
        if k not in resident:
            misses += tix[i] >= warm
            if len(resident) >= slots:
                while True:
                    nu, kk = heapq.heappop(heap)
                    if resident.get(kk) == -nu:
                        del resident[kk]
                        break
        resident[k] = int(nxt[i])
        heapq.heappush(heap, (-int(nxt[i]), k))
    return misses / max(n_tokens - warm, 1)


def evaluate(path, slots=(952, 1508), warm=20, topk=8, n_experts=288):
    toks = tokens_of(load(path, topk))
    keys, tix = accesses(toks, topk, n_experts)
    rows = []
    for s in slots:
        rows.append({"slots": s, "lru": round(float(lru_misses(toks, s, warm, topk, n_experts)), 2),
                     "belady": round(float(belady_misses(keys, tix, s, warm, len(toks))), 2)})
    return {"tokens": len(toks), "measured_tokens": max(len(toks) - warm, 0), "warm": warm,
            "layers": len({layer for tok in toks for layer, _ in tok}), "misses_per_token": rows}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("trace")
    ap.add_argument("--slots", type=int, nargs="+", default=[952, 1508])
    ap.add_argument("--warm", type=int, default=20)
    ap.add_argument("--topk", type=int, default=8)
    ap.add_argument("--experts", type=int, default=288)
    a = ap.parse_args()
    print(json.dumps(evaluate(a.trace, a.slots, a.warm, a.topk, a.experts)))


if __name__ == "__main__":
    main()
