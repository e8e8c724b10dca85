"""Calibrated Zipf routing for the synthetic skewed workloads (BASELINE configs 3 and 5).

Target: expert popularity Zipf(s), i.e. the probability that the expert of popularity rank r
(1-based) is among a token's top-k is p_r = min(1, c * r**-s) with c fixed by sum_r p_r = k
(a top-k selection picks k distinct experts, so no probability can exceed 1: at s = 1.1 over
288 experts and k = 8 only rank 1 saturates). For config 5, additionally a token-to-token
reuse of about 70%: the fraction of a token's experts that the previous token of the same layer
also chose.

Model of the router: the selection score is sigmoid(z_e) + b_e with z = W x. Rows of W are
i.i.d. N(0, sigma^2) and |x|^2 is close to its mean, so for one token the z_e are i.i.d.
N(0, sigma^2 |x|^2) = N(0, 1) at BASELINE's "router logits ~ N(0, 1)". Popularity is therefore a
function of the bias vector alone, and the bias b(rank) that makes it Zipf(s) is the same curve
for every layer (each layer permutes it over its experts). With inputs that evolve as
x <- rho x + sqrt(1 - rho^2) n, the logits follow the same AR(1) per expert, which leaves the
popularity unchanged and sets the reuse; rho is chosen for the target reuse.

calibrate() fits b by a damped fixed-point iteration on the log-frequency error over a seeded
sample of logits, then bisects rho; the result for the released shapes is stored in
zipf_table.json beside this file (python -m glm53h.zipf rewrites it), so workloads do not pay
the fitting time."""
from __future__ import annotations

import json
import os

import numpy as np

TABLE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "zipf_table.json")


def target(NE, K, s):
    """p_r = min(1, c r^-s), sum = K."""
    r = np.arange(1, NE + 1, dtype=np.float64)
    lo, hi = 0.0, float(K) * 4
    for _ in range(200):
        c = 0.5 * (lo + hi)
        if np.minimum(1.0, c * r ** -s).sum() > K:
            hi = c
        else:
            lo = c
    return np.minimum(1.0, lo * r ** -s)


def _select(sig, b, K):
    sc = sig + b
    sel = np.argpartition(-sc, K, axis=1)[:, :K]
    m = np.zeros(sc.shape, bool)
    np.put_along_axis(m, sel, True, 1)
    return m


def frequencies(b, K, M=20000, seed=7, rho=0.0):
    """(selection frequency per expert, reuse) of scores sigmoid(z) + b over M tokens of AR(1)
    logits."""
    rng = np.random.default_rng(seed)
    NE = len(b)
    z = rng.standard_normal(NE)
    Z = np.empty((M, NE))
    a = np.sqrt(1 - rho * rho)
    for t in range(M):
        z = rho * z + a * rng.standard_normal(NE)
        Z[t] = z
    m = _select(1 / (1 + np.exp(-Z)), b, K)
    return m.mean(0), (m[1:] & m[:-1]).sum() / (K * (M - 1))


def calibrate(NE=288, K=8, s=1.1, reuse=0.70, M=20000, iters=150, seed=7):
    p = target(NE, K, s)
    rng = np.random.default_rng(seed)
    sig = 1 / (1 + np.exp(-rng.standard_normal((M, NE))))
    b = -0.3 * np.log(np.arange(1, NE + 1))
    for _ in range(iters):
        f = _select(sig, b, K).mean(0)
        b += 0.03 * np.clip(np.log(np.maximum(p, 1e-6)) - np.log(np.maximum(f, 0.5 / M)), -1, 1)
    f = _select(sig, b, K).mean(0)
    lo, hi = 0.0, 0.99
    for _ in range(14):
        rho = 0.5 * (lo + hi)
        if frequencies(b, K, M // 2, seed + 1, rho)[1] < reuse:
            lo = rho
        else:
            hi = rho
    rho = 0.5 * (lo + hi)
    return {"NE": NE, "K": K, "s": s, "reuse": reuse, "rho": round(rho, 4),
            "bias_by_rank": [round(float(v), 6) for v in b - b[0]],
            "fit_max_rel_err_top100": float(np.max(np.abs(f[:100] / p[:100] - 1)))}


def table(NE, K, s):
    """The stored calibration for (NE, K, s), or a fresh one (slow) when none is stored."""
    if os.path.exists(TABLE):
        with open(TABLE) as fh:
            for t in json.load(fh):
                if t["NE"] == NE and t["K"] == K and abs(t["s"] - s) < 1e-9:
                    return t
    return calibrate(NE, K, s)


def slope(freq_by_rank, lo=2, hi=200):
    """Least-squares exponent of frequency against rank over ranks [lo, hi] (1-based)."""
    r = np.arange(1, len(freq_by_rank) + 1)
    keep = (r >= lo) & (r <= hi) & (freq_by_rank > 0)
    return float(np.polyfit(np.log(r[keep]), np.log(freq_by_rank[keep]), 1)[0])


if __name__ == "__main__":
    out = [calibrate(288, 8, 1.1)]
    with open(TABLE, "w") as fh:
        json.dump(out, fh, indent=0)
    for t in out:
        print(t["NE"], t["K"], t["s"], "rho", t["rho"], "fit err", t["fit_max_rel_err_top100"])
