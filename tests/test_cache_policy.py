"""The HBM expert cache's policy (LRU victim choice, pins, getmany, the hint queue and its
cancellation rules, background reads) against the reference's own cache
(src/cache/glm53f_cache.c) on scripted traces: every per-call output (hit or miss, slot index,
queue contents after each hint, slots of background reads) and the final statistics must be
identical. CPU only: the policy is the library's host code, g53h_lru_trace."""
import ctypes as C
import os

import numpy as np
import pytest

import glm53h
import cache_traces as CT
import oracle_lib as O

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = np.load(os.path.join(HERE, "golden", "cache_traces.npz"))


def lib_trace(ops, nslot):
    L = glm53h.lib()
    f = L.g53h_lru_trace
    f.restype = C.c_int
    f.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p]
    ops = np.asarray(ops, np.int32)
    out = np.zeros(200000, np.int32)
    st = np.zeros(6, np.int64)
    n = f(CT.N_LAYERS, CT.N_EXPERTS, nslot, ops.ctypes.data, len(ops), out.ctypes.data, len(out), st.ctypes.data)
    assert n >= 0
    return out[:n], st


@pytest.mark.parametrize("k", range(len(CT.CASES)))
def test_policy_matches_reference_golden(k):
    seed, steps, nslot, hints, gm = CT.CASES[k]
    ops = CT.trace(seed, steps, nslot, hints, gm)
    assert np.array_equal(np.asarray(ops, np.int32), GOLD[f"t{k}_ops"]), "trace generator changed"
    out, st = lib_trace(ops, nslot)
    want = GOLD[f"t{k}_out"]
    assert len(out) == len(want)
    if not np.array_equal(out, want):
        i = int(np.argmax(out != want))
        raise AssertionError(f"first difference at output {i}: got {out[max(0, i - 6):i + 6]}, "
                             f"want {want[max(0, i - 6):i + 6]}")
    assert np.array_equal(st, GOLD[f"t{k}_stats"])


def test_policy_matches_live_reference():
    """Fresh traces (other seeds) against the compiled reference cache, where it is built."""
    if not O.have_ref() or not hasattr(O.ref(), "ref_cache_trace"):
        pytest.skip("oracle/_ref reference cache not built here")
    import sys
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import make_cache_traces as MT
    for seed in range(100, 112):
        nslot = [3, 4, 6, 9, 13, 30][seed % 6]
        ops = CT.trace(seed, 7, nslot, seed % 3 != 0, seed % 2 == 0)
        want, wst = MT.ref_trace(O.ref(), ops, nslot)
        out, st = lib_trace(ops, nslot)
        assert np.array_equal(out, want), seed
        assert np.array_equal(st, wst), seed
    for seed in range(200, 206):                 # long traces: deep eviction heaps, long queues
        nslot = [3, 5, 8, 12, 20, 30][seed % 6]
        ops = CT.trace(seed, 80, nslot, True, seed % 2 == 0)
        want, wst = MT.ref_trace(O.ref(), ops, nslot)
        out, st = lib_trace(ops, nslot)
        assert np.array_equal(out, want), seed
        assert np.array_equal(st, wst), seed


def test_lru_victim_order_closed_form():
    """With no pins, no hints and distinct keys, a cache of n slots evicts in first-in order:
    the (n+1)-th distinct expert takes slot 0, the next slot 1, ... (a property the policy must
    have regardless of the reference)."""
    n = 4
    ops = []
    keys = [(1, e) for e in range(6)] + [(2, e) for e in range(6)]
    for L, e in keys:
        ops += [1, L, e, 2, L, e]
    out, st = lib_trace(ops, n)
    slots = out.reshape(-1, 3)[:, 2]
    assert list(slots) == [i % n for i in range(len(keys))]
    assert st[1] == len(keys) and st[2] == len(keys) - n and st[0] == 0
