"""Write tests/golden/protocol.npz: the reference's expert-source protocol (hints, getmany, get,
release, in call order) and outputs for seeded config-1-shaped layers, recorded from the
reference's own glm53f_moe (src/core/glm53f_ops.c:1144-1362, compiled into
oracle/_ref/libglm53f_ref.so) through oracle/ref_shim.c's recording source.

Cases (name: tokens, prefetch_n, prefill_next, hint, getmany, environment):
  t1   decode, 4 tokens one at a time, prediction of 6
  t5   a chunk of 5 tokens, prefill prediction voted (prefill_next)
  t70  70 tokens: two chunks (64 + 6), prefill prediction voted
  nopf 70 tokens without prefetch: getmany batches of 16, no hints
  nopp 70 tokens with GLM53F_NO_PREFILL_PREFETCH (prefill hints off, decode unaffected)
  pp3  70 tokens with GLM53F_PREFILL_PRED=3 (3 predictions per token, vote without prefill_next)
  drop 5 tokens, experts 3 and 11 failing to load

Usage (build container, /root/reference present): make -C oracle && python tests/golden/make_protocol.py
"""
import json
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "glm-5.3-flash-in-c_amd"))

CASES = {  # name: (tokens, one token per call, prefetch_n, prefill_next, hint, getmany, env, drop)
    "t1": (4, True, 6, 0, True, True, {}, ()),
    "t5": (5, False, 6, 1, True, True, {}, ()),
    "t70": (70, False, 6, 1, True, True, {}, ()),
    "nopf": (70, False, 0, 0, False, True, {}, ()),
    "nopp": (70, False, 6, 1, True, True, {"GLM53F_NO_PREFILL_PREFETCH": "1"}, ()),
    "pp3": (70, False, 6, 0, True, True, {"GLM53F_PREFILL_PRED": "3"}, ()),
    "drop": (5, False, 6, 1, True, True, {}, (3, 11)),
}
LAYER = 2


def inputs(name):
    import glm53h.synth as S
    tokens = CASES[name][0]
    sp = S.spec(1, seed=21)
    nsp = S.spec(1, seed=21, layer=LAYER + 1)
    W, b = S.router_host(S.spec(1, seed=21, layer=LAYER)), S.bias_host(S.spec(1, seed=21, layer=LAYER))
    Wn, bn = S.router_host(nsp), S.bias_host(nsp)
    ex = {e: S.expert_host(sp, e) for e in range(sp.NE)}
    sh = S.expert_host(sp, "shared")
    x = S.x_host(sp, tokens, batch=7)
    return sp, W, b, Wn, bn, ex, sh, x


def run_case(name):
    import oracle_lib as O
    tokens, single, pf, pn, hint, gm, env, drop = CASES[name]
    sp, W, b, Wn, bn, ex, sh, x = inputs(name)
    mats = {e: m for e, m in ex.items() if e not in drop}
    if single:
        outs, logs = [], []
        for t in range(tokens):
            o, lg = O.ref_proto(sp, x[t:t + 1], W, b, mats, sh, LAYER, Wn, bn, pf, pn, hint, gm)
            outs.append(o)
            logs.append(lg)
        return np.concatenate(outs), np.concatenate(logs)
    return O.ref_proto(sp, x, W, b, mats, sh, LAYER, Wn, bn, pf, pn, hint, gm)


def main():
    if len(sys.argv) > 2 and sys.argv[1] == "--case":        # one case in a fresh process (its environment)
        out, log = run_case(sys.argv[2])
        np.savez(sys.argv[3], out=out, log=log)
        return
    g = {}
    for name, case in CASES.items():
        tmp = os.path.join(HERE, f"_proto_{name}.npz")
        env = dict(os.environ)
        env.update(case[6])
        subprocess.run([sys.executable, __file__, "--case", name, tmp], check=True, env=env)
        d = np.load(tmp)
        g[f"{name}_out"], g[f"{name}_log"] = d["out"], d["log"]
        os.remove(tmp)
        print(f"{name}: {len(d['log'])} ints of protocol")
    g["cases"] = np.frombuffer(json.dumps({k: [v[0], v[1], v[2], v[3], v[4], v[5], v[6], list(v[7])]
                                            for k, v in CASES.items()}).encode(), np.uint8)
    np.savez_compressed(os.path.join(HERE, "protocol.npz"), **g)


if __name__ == "__main__":
    main()
