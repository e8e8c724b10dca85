"""The drop-in's GLM53F_ROUTE_TOP16 trace against the reference's on the same inputs
(src/core/glm53f_ops.c:1044-1080: one line per decode MoE layer, the layer, then the 16 best
experts by score + bias, id:%.6g of the pre-normalisation sigmoid, the lower index first among
equal values). tests/golden/top16.npz holds the lines the compiled reference wrote
(tests/golden/make_top16.py: 3 config-2-shaped layers, 4 decode tokens each, tied choices on
layer 2). The drop-in runs the same calls in a child process, since both sides read the switch
once per process, and its file must equal the reference's line for line: ids exactly, scores as
the same %.6g text. This is what makes the cache-policy evaluation on the drop-in's trace
comparable with the reference's own tool."""
import ctypes as C
import os
import subprocess
import sys
import tempfile

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_top16 as MT  # noqa: E402

pytestmark = pytest.mark.gpu


def run_dropin():
    import glm53h
    import glm53h.synth as S
    from test_gpu_parity import HostSrc, cfg_struct, fmat
    L = glm53h.init(0)
    sh = S.expert_host(S.spec(2, seed=31), "shared")
    for layer in MT.LAYERS:
        sp, W, b, x = MT.inputs(layer)
        cf = cfg_struct(dict(E=sp.E, I=sp.I, NE=sp.NE, K=sp.K, routed_scale=sp.routed_scale,
                             norm_topk=sp.norm_topk, limit=sp.limit, br=sp.br, bc=sp.bc))
        cf.n_layers = 3
        src = HostSrc(cf, {}, drop=range(sp.NE))        # no expert present: every fetch drops
        w = glm53h.Glm53fMoeW()
        w.gate, w.bias = W.ctypes.data, b.ctypes.data
        (gw, gs), (uw, us), (dw, ds) = sh
        w.sh_gate, w.sh_up = fmat(gw, gs, sp.I, sp.E, sp.br, sp.bc), fmat(uw, us, sp.I, sp.E, sp.br, sp.bc)
        w.sh_down = fmat(dw, ds, sp.E, sp.I, sp.br, sp.bc)
        w.src = C.pointer(src.src)
        w.layer = layer
        for t in range(MT.TOKENS):
            o = np.zeros((1, sp.E), np.float32)
            xt = np.ascontiguousarray(x[t:t + 1])
            L.glm53f_moe(o.ctypes.data, xt.ctypes.data, C.byref(w), C.byref(cf), 1, None)
        L.glm53f_forget_host_weights()


def test_route_top16_trace_equals_reference():
    want = [str(v) for v in np.load(os.path.join(HERE, "golden", "top16.npz"))["lines"]]
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "top16.txt")
        env = dict(os.environ, GLM53F_ROUTE_TOP16=path)
        print("[gpu] drop-in routing trace in a child process", flush=True)
        r = subprocess.run([sys.executable, "-u", __file__], env=env, capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
        with open(path) as f:
            got = f.read().splitlines()
    assert len(got) == len(want), (len(got), len(want))
    for i, (g, w) in enumerate(zip(got, want)):
        assert g == w, f"line {i}:\n got  {g}\n want {w}"
    # the tied group (experts 5, 17, 200 on layer 2) appears, in index order
    tied = [ln for ln in got if ln.startswith("2 ") and " 5:" in ln]
    assert tied and all(ln.index(" 5:") < ln.index(" 17:") < ln.index(" 200:") for ln in tied)


if __name__ == "__main__":
    sys.path.insert(0, os.path.join(os.path.dirname(HERE), "glm-5.3-flash-in-c_amd"))
    sys.path.insert(0, HERE)
    run_dropin()
    print("ok", flush=True)
