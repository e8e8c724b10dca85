"""Minimal reader of the reference's glm_tiny fixture (tests/golden/glm_tiny/model.safetensors,
copied as data from the reference's tests/fixtures/glm_tiny/). The safetensors layout is an
8-byte little-endian header length, a JSON header of {name: {dtype, shape, data_offsets}},
then the raw tensor bytes; nothing in the file is executed."""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
TINY = os.path.join(HERE, "glm_tiny")

_DT = {"F8_E4M3": np.uint8, "F32": np.float32, "BF16": np.uint16}


def load(path=os.path.join(TINY, "model.safetensors")):
    with open(path, "rb") as f:
        raw = f.read()
    n = int.from_bytes(raw[:8], "little")
    hdr = json.loads(raw[8:8 + n])
    base = 8 + n
    out = {}
    for k, v in hdr.items():
        if k == "__metadata__":
            continue
        a, b = v["data_offsets"]
        out[k] = np.frombuffer(raw[base + a:base + b], _DT[v["dtype"]]).reshape(v["shape"]).copy()
    return out


def config():
    with open(os.path.join(TINY, "config.json")) as f:
        c = json.load(f)
    t = c["text_config"]
    return dict(E=t["hidden_size"], I=t["moe_intermediate_size"], NE=t["n_routed_experts"],
                K=t["num_experts_per_tok"], routed_scale=t["routed_scaling_factor"],
                norm_topk=int(t["norm_topk_prob"]), limit=t["swiglu_limit"],
                br=c["quantization_config"]["weight_block_size"][0],
                bc=c["quantization_config"]["weight_block_size"][1],
                moe_layers=[i for i, m in enumerate(t["mlp_layer_types"]) if m == "sparse"])


def layer(tensors, L):
    """(router fp32 [NE][E] widened from bf16, bias, {e: [(w, s)] x 3}, shared [(w, s)] x 3)."""
    p = f"model.language_model.layers.{L}.mlp."
    router = (tensors[p + "gate.weight"].astype(np.uint32) << 16).view(np.float32)
    bias = tensors[p + "gate.e_score_correction_bias"].astype(np.float32)

    def mats(q):
        return [(np.ascontiguousarray(tensors[q + m + "_proj.weight"]).reshape(-1),
                 np.ascontiguousarray(tensors[q + m + "_proj.weight_scale_inv"]).reshape(-1))
                for m in ("gate", "up", "down")]

    experts = {}
    e = 0
    while p + f"experts.{e}.gate_proj.weight" in tensors:
        experts[e] = mats(p + f"experts.{e}.")
        e += 1
    return np.ascontiguousarray(router), bias, experts, mats(p + "shared_experts.")
