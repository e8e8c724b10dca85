"""The drop-in's expert-source protocol, call for call, against the reference's.

tests/golden/protocol.npz holds, per case, the reference glm53f_moe's output and the exact sequence
of hint / getmany / get / release calls it makes on its source (src/core/glm53f_ops.c:1144-1362,
recorded by oracle/ref_shim.c, written by tests/golden/make_protocol.py). Here the drop-in runs the
same layer on the GPU behind a host-memory source that logs the same way; both the log and the
output (bit for bit) must match. Cases that set GLM53F_NO_PREFILL_PREFETCH / GLM53F_PREFILL_PRED
(read once per process, as the reference does) run in a child process."""
import ctypes as C
import json
import os
import subprocess
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_protocol as MP  # noqa: E402  (inputs and case table of the fixture)

pytestmark = pytest.mark.gpu
GOLD = np.load(os.path.join(HERE, "golden", "protocol.npz"))


def say(*a):
    print("[gpu]", *a, flush=True)


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


class LogSrc:
    """A Glm53fExpertSrc serving host memory that logs like the reference recorder:
    [1, L, e] get, [2, L, e] release, [3, L, n, ids] getmany, [4, L, n, ids] hint."""

    def __init__(self, glm53h, cf, experts, hint=True, getmany=True):
        self.g, self.cf, self.ex, self.log = glm53h, cf, experts, []
        self.src = glm53h.Glm53fExpertSrc()
        self._fns = [glm53h.GET_FN(self.get), glm53h.RELEASE_FN(self.release)]
        self.src.get, self.src.release = self._fns
        if getmany:
            self._fns.append(glm53h.GETMANY_FN(self.getmany))
            self.src.getmany = self._fns[-1]
        if hint:
            self._fns.append(glm53h.HINT_FN(self.hint))
            self.src.hint = self._fns[-1]

    def mat(self, w, s, rows, cols):
        br, bc = self.cf.fp8_block_r, self.cf.fp8_block_c
        return self.g.Glm53fMat(w.ctypes.data, s.ctypes.data, self.g.GLM53F_WF8, rows, cols, br, bc, (cols + bc - 1) // bc)

    def get(self, selfp, layer, e, q):
        self.log += [1, layer, e]
        if e not in self.ex:
            return -1
        (gw, gs), (uw, us), (dw, ds) = self.ex[e]
        E, I = self.cf.hidden, self.cf.moe_inter
        q[0].gate, q[0].up, q[0].down = self.mat(gw, gs, I, E), self.mat(uw, us, I, E), self.mat(dw, ds, E, I)
        return 0

    def release(self, selfp, layer, e):
        self.log += [2, layer, e]

    def getmany(self, selfp, layer, ids, n):
        self.log += [3, layer, n] + [ids[i] for i in range(n)]
        return 0

    def hint(self, selfp, layer, ids, n):
        self.log += [4, layer, n] + [ids[i] for i in range(n)]


def run_case(name):
    """The drop-in on one fixture case: (output, log)."""
    import glm53h
    glm53h.init(0)
    L = glm53h.lib()
    tokens, single, pf, pn, hint, gm, env, drop = MP.CASES[name]
    sp, W, b, Wn, bn, ex, sh, x = MP.inputs(name)
    cf = glm53h.Glm53fCfg()
    cf.hidden, cf.moe_inter, cf.n_experts, cf.topk, cf.n_shared = sp.E, sp.I, sp.NE, sp.K, 1
    cf.routed_scale, cf.norm_topk, cf.swiglu_limit = sp.routed_scale, sp.norm_topk, sp.limit
    cf.fp8_block_r, cf.fp8_block_c = sp.br, sp.bc
    cf.n_layers = MP.LAYER + 2
    src = LogSrc(glm53h, cf, {e: m for e, m in ex.items() if e not in drop}, hint, gm)
    arrs = [np.ascontiguousarray(a, np.float32) for a in (W, b, Wn, bn)]
    w = glm53h.Glm53fMoeW()
    w.gate, w.bias, w.next_gate, w.next_bias = [a.ctypes.data for a in arrs]
    (gw, gs), (uw, us), (dw, ds) = sh
    w.sh_gate, w.sh_up, w.sh_down = src.mat(gw, gs, sp.I, sp.E), src.mat(uw, us, sp.I, sp.E), src.mat(dw, ds, sp.E, sp.I)
    w.src = C.pointer(src.src)
    w.layer, w.prefetch_n, w.prefill_next = MP.LAYER, pf, pn
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    steps = [(t, t + 1) for t in range(tokens)] if single else [(0, tokens)]
    for t0, t1 in steps:
        o = np.zeros((t1 - t0, sp.E), np.float32)
        L.glm53f_moe(o.ctypes.data, x[t0:t1].ctypes.data, C.byref(w), C.byref(cf), t1 - t0, None)
        out[t0:t1] = o
    L.glm53f_forget_host_weights()
    return out, np.array(src.log, np.int32)


def check_case(name):
    out, log = run_case(name)
    want = GOLD[f"{name}_log"]
    if not np.array_equal(log, want):
        n = min(len(log), len(want))
        d = next((i for i in range(n) if log[i] != want[i]), n)
        raise AssertionError(f"{name}: protocol differs at int {d}: got {log[max(0, d - 6):d + 12].tolist()} "
                             f"want {want[max(0, d - 6):d + 12].tolist()} (lengths {len(log)} / {len(want)})")
    assert same(out, GOLD[f"{name}_out"]), f"{name}: output differs from the reference"


@pytest.mark.parametrize("name", [n for n, c in MP.CASES.items() if not c[6]])
def test_protocol_matches_reference(name):
    say("drop-in protocol case", name)
    check_case(name)


def test_protocol_env_switches():
    """GLM53F_NO_PREFILL_PREFETCH and GLM53F_PREFILL_PRED, each in a fresh process."""
    for name, case in MP.CASES.items():
        if not case[6]:
            continue
        say("drop-in protocol case", name, "in a child process with", case[6])
        env = dict(os.environ)
        env.update(case[6])
        r = subprocess.run([sys.executable, "-u", __file__, name], env=env, capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, f"{name}: {r.stdout[-2000:]}\n{r.stderr[-2000:]}"


def test_fixture_case_table():
    """The case table the fixture was written with is the one the test runs."""
    rec = json.loads(bytes(GOLD["cases"]).decode())
    assert rec == {k: [v[0], v[1], v[2], v[3], v[4], v[5], v[6], list(v[7])] for k, v in MP.CASES.items()}


if __name__ == "__main__":
    sys.path.insert(0, os.path.join(os.path.dirname(HERE), "glm-5.3-flash-in-c_amd"))
    check_case(sys.argv[1])
    print("ok", sys.argv[1], flush=True)
