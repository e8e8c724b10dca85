"""Trace-driven cache policy evaluation (glm53h.route_trace) on the CPU: the Belady bound
against exhaustive search for the fewest misses on small traces, the library's LRU replay
(g53h_lru_trace, the HBM cache's own policy) against a plain LRU, closed forms on cyclic
traces, and the GLM53F_ROUTE_TOP16 line format (src/core/glm53f_ops.c:1044-1080)."""
import functools
import os

import numpy as np

import glm53h.route_trace as RT


def fewest_misses(seq, cap):
    """Exhaustive search over every eviction choice: the minimum number of misses."""
    @functools.lru_cache(maxsize=None)
    def go(i, cache):
        if i == len(seq):
            return 0
        k = seq[i]
        if k in cache:
            return go(i + 1, cache)
        if len(cache) < cap:
            return 1 + go(i + 1, cache | frozenset([k]))
        return 1 + min(go(i + 1, (cache - frozenset([v])) | frozenset([k])) for v in cache)
    return go(0, frozenset())


def test_belady_is_optimal_on_small_traces():
    rng = np.random.default_rng(0)
    for trial in range(60):
        n, nk, cap = int(rng.integers(4, 13)), int(rng.integers(2, 7)), int(rng.integers(1, 4))
        seq = rng.integers(0, nk, n)
        got = RT.belady_misses(seq, np.zeros(n, np.int64), cap, 0, 1)
        assert got == fewest_misses(tuple(int(v) for v in seq), cap), (seq, cap)


def test_cyclic_trace_closed_forms():
    """Cycling over c + 1 keys with c slots: LRU misses every access; the optimum misses the
    first c + 1 accesses and then once per c accesses (rate 1/c), exact against exhaustive
    search on a short cycle."""
    c, rounds = 5, 40
    seq = np.tile(np.arange(c + 1), rounds)
    n = len(seq)
    lru = RT.lru_misses_py(seq, np.zeros(n, np.int64), c, 0, 1)
    bel = RT.belady_misses(seq, np.zeros(n, np.int64), c, 0, 1)
    assert lru == n
    rest = n - (c + 1)
    assert rest // c <= bel - (c + 1) <= -(-rest // c)
    short = np.tile(np.arange(4), 4)
    assert RT.belady_misses(short, np.zeros(16, np.int64), 3, 0, 1) == fewest_misses(tuple(short.tolist()), 3)


def write_trace(path, steps):
    with open(path, "w") as f:
        for layer, cand in steps:
            f.write("%d" % layer + "".join(" %d:%.6g" % (e, s) for e, s in cand) + "\n")


def random_steps(rng, n_tokens, n_layers, ne, k, skew=1.1):
    p = np.arange(1, ne + 1, dtype=np.float64) ** -skew
    p /= p.sum()
    steps = []
    for _ in range(n_tokens):
        for layer in range(n_layers):
            ids = rng.choice(ne, 16, replace=False, p=p)
            steps.append((layer, [(int(e), float(rng.random())) for e in ids]))
    return steps


def test_library_lru_replay_equals_plain_lru(tmp_path):
    rng = np.random.default_rng(1)
    steps = random_steps(rng, 30, 6, 40, 8)
    path = os.path.join(tmp_path, "t.txt")
    write_trace(path, steps)
    toks = RT.tokens_of(RT.load(path))
    assert len(toks) == 30 and all(len(t) == 6 for t in toks)
    keys, tix = RT.accesses(toks, 8, 40)
    for slots in (8, 20, 64, 150, 240):
        lib_ = RT.lru_misses(toks, slots, 5, 8, 40)
        py = RT.lru_misses_py(keys, tix, slots, 5, len(toks))
        bel = RT.belady_misses(keys, tix, slots, 5, len(toks))
        assert abs(lib_ - py) < 1e-12, (slots, lib_, py)
        assert bel <= py


def test_format_round_trip_and_evaluate(tmp_path):
    rng = np.random.default_rng(2)
    steps = random_steps(rng, 25, 4, 288, 8)
    path = os.path.join(tmp_path, "t.txt")
    write_trace(path, steps)
    back = RT.load(path)
    assert [(l, [e for e, _ in c]) for l, c in back] == [(l, [e for e, _ in c]) for l, c in steps]
    r = RT.evaluate(path, slots=(16, 200), warm=5)
    assert r["tokens"] == 25 and r["layers"] == 4
    for row in r["misses_per_token"]:
        assert 0 <= row["belady"] <= row["lru"] <= 4 * 8
