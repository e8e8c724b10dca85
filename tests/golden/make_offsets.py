"""Write tests/golden/offsets.json: sizeof and offsetof of every field of the structs the
reference's callers share with this library (the expert-forward boundary, include/glm53f/
glm53f.h:48-247; the cache, src/cache/glm53f_cache.h:44-96; the safetensors reader,
src/io/glm53f_st.h:27-58), compiled with gcc against the reference's own headers.
tests/test_abi_offsets.py compiles the same probe against include/ and compares.

Usage (build container, /root/reference present): python tests/golden/make_offsets.py"""
import json
import os
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
REF = os.environ.get("GLM53F_REF", "/root/reference")

STRUCTS = {
    "Glm53fCfg": ["hidden", "n_layers", "vocab", "rms_eps", "hc_mult", "hc_iters", "hc_eps", "kda_heads",
                  "kda_head_dim", "conv_k", "gate_lb", "n_heads", "q_lora", "kv_lora", "qk_nope", "v_head",
                  "index_topk", "index_kpool", "index_heads", "index_dim", "index_tail", "n_experts", "topk",
                  "n_shared", "moe_inter", "dense_inter", "routed_scale", "norm_topk", "swiglu_limit",
                  "fp8_block_r", "fp8_block_c", "is_mla", "is_dense", "eos", "n_eos"],
    "Glm53fMat": ["w", "s", "dt", "rows", "cols", "br", "bc", "scols"],
    "Glm53fExpertQ": ["gate", "up", "down"],
    "Glm53fExpertSrc": ["get", "getmany", "release", "hint", "ctx"],
    "Glm53fMoeW": ["gate", "bias", "sh_gate", "sh_up", "sh_down", "src", "next_gate", "next_bias", "ahead_gate",
                   "ahead_bias", "prefetch_n", "prefill_next", "layer"],
    "Glm53fCache": ["src", "st", "cfg", "n_layers", "n_experts", "arena", "slot_bytes", "nslot", "i4", "raw_bytes",
                    "stage", "stage_busy", "nstage", "stage_free", "i4_fd", "i4_layers", "slot_of", "inflight_of",
                    "key_of", "pins", "prefetched", "used_at", "ref", "pad", "clock", "mu", "landed", "work",
                    "n_io", "io", "stop", "queue", "qcap", "qlen", "hint_floor", "last_hint", "queued", "hits",
                    "misses", "evictions", "bytes_read", "prefetch_reads", "load_seconds", "bg_reads", "bg_bytes",
                    "bg_used"],
    "Glm53fSt": ["fd", "dfd", "path", "nshard", "t", "nt", "bucket", "nbucket", "strpool", "strcap", "strlen_"],
    "Glm53fTensor": ["name", "shard", "dtype", "ndim", "shape", "off", "nbytes"],
}


def probe_source():
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "glm53f.h"', '#include "glm53f_st.h"',
             '#include "glm53f_cache.h"', 'int main(void) {', '    printf("{");']
    first = True
    for s, fields in STRUCTS.items():
        sep = "" if first else ","
        first = False
        lines.append(f'    printf("{sep}\\"{s}\\": {{\\"sizeof\\": %zu", sizeof({s}));')
        for f in fields:
            lines.append(f'    printf(", \\"{f}\\": %zu", offsetof({s}, {f}));')
        lines.append('    printf("}");')
    lines += ['    printf("}\\n");', '    return 0;', '}']
    return "\n".join(lines) + "\n"


def offsets(include_dirs):
    """Compile and run the probe against the given include directories."""
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "probe.c"), os.path.join(d, "probe")
        with open(src, "w") as f:
            f.write(probe_source())
        cmd = ["gcc", "-std=gnu99", "-O0", "-o", exe, src, "-lpthread"] + [f"-I{p}" for p in include_dirs]
        subprocess.run(cmd, check=True)
        return json.loads(subprocess.run([exe], check=True, capture_output=True, text=True).stdout)


def main():
    inc = [os.path.join(REF, p) for p in ("include/glm53f", "src/io", "src/cache", "third_party")]
    got = offsets(inc)
    with open(os.path.join(HERE, "offsets.json"), "w") as f:
        json.dump(got, f, indent=1, sort_keys=True)
    print({k: v["sizeof"] for k, v in got.items()})


if __name__ == "__main__":
    sys.exit(main())
