"""Next-layer prediction on the GPU (g53h_route_topn_batch, g53h_vote) against the oracle's
restatement of the reference's route_topn (src/core/glm53f_ops.c:1021-1042) and the prefill
vote (src/core/glm53f_ops.c:1206-1225); and the drop-in's abort on kernel error flags."""
import ctypes as C
import os
import subprocess
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
for _p in (HERE, os.path.join(os.path.dirname(HERE), "glm-5.3-flash-in-c_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import glm53h  # noqa: E402
import glm53h.synth as S  # noqa: E402
import oracle_lib as O  # noqa: E402
from glm53h import DevBuf, check  # noqa: E402

pytestmark = pytest.mark.gpu


def say(*a):
    print("[gpu]", *a, flush=True)


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


def topn_oracle(x, W, b, n):
    Lo = O.oracle()
    Lo.or_route_topn.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int]
    NE, E = W.shape
    out = np.zeros((x.shape[0], n), np.int32)
    W, b = np.ascontiguousarray(W, np.float32), np.ascontiguousarray(b, np.float32)
    for t in range(x.shape[0]):
        xt = np.ascontiguousarray(x[t], np.float32)
        Lo.or_route_topn(out[t].ctypes.data, n, xt.ctypes.data, W.ctypes.data, b.ctypes.data, NE, E)
    return out


def topn_gpu(L, x, W, b, n, bf16=False, scores=False):
    T, E = x.shape
    NE = W.shape[0]
    if bf16:
        gate = DevBuf.from_array((np.ascontiguousarray(W, np.float32).view(np.uint32) >> 16).astype(np.uint16))
    else:
        gate = DevBuf.from_array(np.ascontiguousarray(W, np.float32))
    xd, bd = DevBuf.from_array(np.ascontiguousarray(x, np.float32)), DevBuf.from_array(np.ascontiguousarray(b, np.float32))
    idx = DevBuf(T * n * 4)
    sc = DevBuf(T * n * 4) if scores else None
    check(L.g53h_route_topn_batch(idx.ptr, sc.ptr if sc else None, n, xd.ptr, T, gate.ptr, int(bf16), bd.ptr, NE, E),
          "g53h_route_topn_batch")
    check(L.g53h_sync(), "sync")
    got = idx.download(np.int32).reshape(T, n)
    return (got, sc.download(np.float32).reshape(T, n)) if scores else got


@pytest.mark.parametrize("bf16", [True, False])
def test_route_topn_batch_config2(L, bf16):
    """64 tokens of config 2 (256 experts, hidden 4096), the 16 best: index for index."""
    sp = S.spec(2)
    W, b, x = S.router_host(sp), S.bias_host(sp), S.x_host(sp, 64, batch=3)
    say("route_topn_batch config 2, T=64, n=16, bf16 router" if bf16 else "fp32 router")
    assert np.array_equal(topn_gpu(L, x, W, b, 16, bf16), topn_oracle(x, W, b, 16))
    one = DevBuf(16 * 4)
    gate = DevBuf.from_array(np.ascontiguousarray(W, np.float32))
    xd, bd = DevBuf.from_array(np.ascontiguousarray(x[5], np.float32)), DevBuf.from_array(b)
    check(L.g53h_route_topn(one.ptr, 16, xd.ptr, gate.ptr, 0, bd.ptr, sp.NE, sp.E), "g53h_route_topn")
    check(L.g53h_sync(), "sync")
    assert np.array_equal(one.download(np.int32), topn_oracle(x[5:6], W, b, 16)[0])


def test_route_topn_scores_are_the_sigmoid(L):
    """score_out holds the chosen experts' sigmoid(W x) before the bias (the top-16 trace)."""
    sp = S.spec(2)
    W, b, x = S.router_host(sp), S.bias_host(sp), S.x_host(sp, 4, batch=4)
    idx, sc = topn_gpu(L, x, W, b, 16, True, scores=True)
    dot = (x.astype(np.float64) @ W.astype(np.float64).T).astype(np.float32)
    want = (1.0 / (1.0 + np.exp(-dot.astype(np.float64)))).astype(np.float32)
    for t in range(4):
        assert np.allclose(sc[t], want[t, idx[t]], rtol=1e-6, atol=0)


def test_route_topn_ties_and_nan(L):
    """All-equal choices pick the lowest indices in order; a NaN at index 0 is taken first, a
    NaN elsewhere never (the strict > of the reference's scan); -inf choices come last."""
    E, NE = 64, 40
    x = np.ones((1, E), np.float32)
    W = np.zeros((NE, E), np.float32)
    cases = [np.zeros(NE, np.float32), np.repeat(np.arange(10, dtype=np.float32), 4)[::-1].copy()]
    for bad in (0, 1, 17):
        bb = np.linspace(0, 1, NE).astype(np.float32)
        bb[bad] = np.nan
        cases.append(bb)
    # -inf choices: taken last, lowest index first; once every value is -inf (taken experts are
    # -inf too) the scan returns expert 0 again
    bb = np.linspace(0, 1, NE).astype(np.float32)
    bb[[3, 9, 30]] = -np.inf
    cases.append(bb)
    for b in cases:
        for n in (1, 7, 40):
            assert np.array_equal(topn_gpu(L, x, W, b, n), topn_oracle(x, W, b, n)), (b, n)
    assert list(topn_gpu(L, x, W, cases[0], 5)[0]) == [0, 1, 2, 3, 4]


def vote_reference_order(ids, NE):
    """Distinct experts by votes descending, ties by first appearance (a stable sort)."""
    votes, first = {}, {}
    for q, e in enumerate(ids.ravel()):
        votes[e] = votes.get(e, 0) + 1
        first.setdefault(e, q)
    return sorted(votes, key=lambda e: (-votes[e], first[e]))


@pytest.mark.parametrize("T,n,NE", [(1, 6, 16), (5, 6, 16), (64, 16, 256), (64, 30, 1024), (3, 4, 8)])
def test_vote_order(L, T, n, NE):
    rng = np.random.default_rng(T * 1000 + n)
    ids = np.stack([rng.choice(min(NE, max(n, NE // 2)), n, replace=False) for _ in range(T)]).astype(np.int32)
    d_ids, d_out = DevBuf.from_array(ids), DevBuf((1 + NE) * 4)
    check(L.g53h_vote(d_out.ptr, d_ids.ptr, T, n, NE), "g53h_vote")
    check(L.g53h_sync(), "sync")
    out = d_out.download(np.int32)
    want = vote_reference_order(ids, NE)
    assert out[0] == len(want) and list(out[1:1 + out[0]]) == want


def test_vote_composes_with_topn_on_fixture_case(L):
    """The device prediction (top-6 per token, then the vote) of the 70-token fixture's first
    chunk equals the reference's hint for the next layer recorded in the fixture."""
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import make_protocol as MP
    sp, W, b, Wn, bn, ex, sh, x = MP.inputs("t70")
    log = np.load(os.path.join(HERE, "golden", "protocol.npz"))["t70_log"]
    i, hints = 0, []
    while i < len(log):
        op, layer = log[i], log[i + 1]
        if op in (1, 2):
            i += 3
            continue
        n = log[i + 2]
        if op == 4 and layer == MP.LAYER + 1:
            hints.append(list(log[i + 3:i + 3 + n]))
        i += 3 + n
    ids = topn_gpu(L, x[:64], Wn, bn, 6)
    d_ids, d_out = DevBuf.from_array(ids), DevBuf((1 + sp.NE) * 4)
    check(L.g53h_vote(d_out.ptr, d_ids.ptr, 64, 6, sp.NE), "g53h_vote")
    check(L.g53h_sync(), "sync")
    out = d_out.download(np.int32)
    assert list(out[1:1 + out[0]]) == hints[0]


# ------------------------------------------------------------- error flags abort ----
def test_dropin_aborts_on_kernel_error_flags():
    """A layer whose kernels raised error flags aborts with the reference's fatal format
    instead of returning the output; each flag word in a fresh process."""
    for word, bits, text in [(1, 8, "reported error flags (decode 0x8"), (0, 1, "a bound or wait was exceeded"),
                             (2, 2, "a wait between waves timed out"), (1, 2, "router selection (NaN scores)")]:
        say("drop-in abort on error word", word, "bits", bits)
        r = subprocess.run([sys.executable, "-u", __file__, str(word), str(bits)], capture_output=True, text=True,
                           timeout=300)
        assert r.returncode == -6, (r.returncode, r.stdout[-1500:], r.stderr[-1500:])
        assert "glm53f: FATAL" in r.stderr and text in r.stderr, r.stderr[-1500:]
        assert "returned" not in r.stdout


def _abort_child(word, bits):
    import test_gpu_parity as P
    L = glm53h.init(0)
    sp = S.spec(1)
    cf = P.cfg_struct(dict(E=sp.E, I=sp.I, NE=sp.NE, K=sp.K, routed_scale=sp.routed_scale, norm_topk=sp.norm_topk,
                           limit=sp.limit, br=sp.br, bc=sp.bc))
    W, b = S.router_host(sp), S.bias_host(sp)
    ex = {e: S.expert_host(sp, e) for e in range(sp.NE)}
    x = S.x_host(sp, 1, batch=1)
    P.dropin_moe(cf, W, b, ex, S.expert_host(sp, "shared"), x)        # clean call: no abort
    check(L.g53h_inject_errors(word, bits), "g53h_inject_errors")
    P.dropin_moe(cf, W, b, ex, S.expert_host(sp, "shared"), x)
    print("returned", flush=True)


if __name__ == "__main__":
    _abort_child(int(sys.argv[1]), int(sys.argv[2]))
