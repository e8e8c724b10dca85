"""Write tests/golden/top16.npz: the routing trace the reference writes with GLM53F_ROUTE_TOP16
set (src/core/glm53f_ops.c:1044-1080: one line per decode MoE layer, the layer, then the 16 best
experts by score + bias as id:%.6g of the pre-normalisation sigmoid), recorded from the
reference's own glm53f_moe (compiled into oracle/_ref/libglm53f_ref.so, driven through
oracle/ref_shim.c) on seeded config-2-shaped layers, 4 decode tokens on each of 3 layers. Layer
2 has tied choices: the router rows and biases of experts 17 and 200 copy expert 5's (its bias
raised to rank the group near the top), so the order among equal values (the lower index first)
is pinned too. No expert is present: the trace
is written before any expert is fetched, and each fetch fails into the reference's drop path.
The reference reads the switch once per process, so the recording runs in a child process.

Usage (build container, /root/reference present): make -C oracle && python tests/golden/make_top16.py
"""
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
LAYERS, TOKENS = (0, 1, 2), 4
TIE = (5, (17, 200))


def inputs(layer):
    """Router (fp32 holding bf16 values), bias and the 4 decode inputs of layer `layer`."""
    sys.path.insert(0, os.path.join(ROOT, "glm-5.3-flash-in-c_amd"))
    import glm53h.synth as S
    sp = S.spec(2, layer=layer, seed=31)
    W, b = S.router_host(sp).copy(), S.bias_host(sp).copy()
    if layer == 2:
        b[TIE[0]] = b.max() + 0.3                       # the tied group ranks near the top
        for e in TIE[1]:
            W[e] = W[TIE[0]]
            b[e] = b[TIE[0]]
    x = S.x_host(sp, TOKENS, batch=9 + layer)
    return sp, W, b, x


def record(path):
    sys.path.insert(0, os.path.dirname(HERE))
    sys.path.insert(0, os.path.join(ROOT, "glm-5.3-flash-in-c_amd"))
    import oracle_lib as O
    import glm53h.synth as S
    sh = S.expert_host(S.spec(2, seed=31), "shared")
    for layer in LAYERS:
        sp, W, b, x = inputs(layer)
        for t in range(TOKENS):
            O.ref_proto(sp, x[t:t + 1], W, b, {}, sh, layer, W, b, 0, 0)


def main():
    if len(sys.argv) > 1 and sys.argv[1] == "--child":
        record(os.environ["GLM53F_ROUTE_TOP16"])
        return
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "top16.txt")
        env = dict(os.environ, GLM53F_ROUTE_TOP16=path)
        subprocess.run([sys.executable, __file__, "--child"], env=env, check=True, stderr=subprocess.DEVNULL)
        with open(path) as f:
            lines = f.read().splitlines()
    assert len(lines) == len(LAYERS) * TOKENS, len(lines)
    np.savez_compressed(os.path.join(HERE, "top16.npz"), lines=np.array(lines))
    print("wrote", len(lines), "lines; first:", lines[0][:120])


if __name__ == "__main__":
    main()
