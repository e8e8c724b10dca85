"""Write tests/golden/cache_traces.npz: the reference's own expert cache (src/cache/
glm53f_cache.c, compiled into oracle/_ref/libglm53f_ref.so from its sources, over the copied
glm_tiny checkpoint) run on the scripted traces of tests/cache_traces.py. Stored per case: the
ops, the slot count, the per-op outputs and the final statistics.

Usage (build container, /root/reference present): make -C oracle && python tests/golden/make_cache_traces.py
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import cache_traces as CT  # noqa: E402
import oracle_lib as O  # noqa: E402


def ref_trace(R, ops, nslot):
    ops = np.asarray(ops, np.int32)
    out = np.zeros(200000, np.int32)
    st = np.zeros(6, np.int64)
    nl, ne = C.c_int(), C.c_int()
    n = R.ref_cache_trace(os.path.join(HERE, "glm_tiny").encode(), nslot, ops.ctypes.data, len(ops),
                          out.ctypes.data, len(out), st.ctypes.data, C.byref(nl), C.byref(ne))
    assert n >= 0, "reference cache trace failed"
    assert (nl.value, ne.value) == (CT.N_LAYERS, CT.N_EXPERTS)
    return out[:n].copy(), st


def main():
    if not O.have_ref():
        sys.exit("oracle/_ref/libglm53f_ref.so is not built")
    R = O.ref()
    g = {}
    for k, (seed, steps, nslot, hints, gm) in enumerate(CT.CASES):
        ops = CT.trace(seed, steps, nslot, hints, gm)
        out, st = ref_trace(R, ops, nslot)
        g[f"t{k}_ops"] = np.asarray(ops, np.int32)
        g[f"t{k}_nslot"] = np.int32(nslot)
        g[f"t{k}_out"] = out
        g[f"t{k}_stats"] = st
        print(f"case {k}: {len(ops)} ints of ops, {len(out)} outputs, stats {st.tolist()}")
    np.savez_compressed(os.path.join(HERE, "cache_traces.npz"), **g)


if __name__ == "__main__":
    main()
