"""Writes small safetensors checkpoints for the checkpoint-reader tests: [8-byte little-endian
header length][JSON header, space-padded to 8 bytes][tensor data]. Tensor data lands in the
order given, so a test controls whether an expert's weights and scales form runs."""
import json
import os

import numpy as np

DT = {np.dtype(np.uint8): "F8_E4M3", np.dtype(np.float32): "F32", np.dtype(np.uint16): "BF16"}
EXPERT = "model.language_model.layers.{}.mlp.experts.{}.{}_proj.{}"


def write_shard(path, tensors):
    """tensors: [(name, array)] in data order."""
    hdr, off = {"__metadata__": {"format": "pt"}}, 0
    for name, a in tensors:
        a = np.ascontiguousarray(a)
        hdr[name] = {"dtype": DT[a.dtype], "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        off += a.nbytes
    h = json.dumps(hdr).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for _, a in tensors:
            f.write(np.ascontiguousarray(a).tobytes())


def expert_tensors(layer, e, mats, shapes, layout):
    """The six tensors of one expert. mats: [(codes, scales)] x 3 (flat); shapes: [(r, c)] x 3.
    layout "runs": three weights then three scales (the released checkpoint's order);
    "interleaved": weight and scale per matrix; "reversed": down, up, gate."""
    br = 128
    ws, ss = [], []
    for m, ((w, s), (r, c)) in enumerate(zip(mats, shapes)):
        p = ("gate", "up", "down")[m]
        ws.append((EXPERT.format(layer, e, p, "weight"), np.asarray(w, np.uint8).reshape(r, c)))
        ss.append((EXPERT.format(layer, e, p, "weight_scale_inv"),
                   np.asarray(s, np.float32).reshape((r + br - 1) // br, -1)))
    if layout == "runs":
        return ws + ss
    if layout == "reversed":
        return ws[::-1] + ss[::-1]
    return [t for pair in zip(ws, ss) for t in pair]


def write_layers(d, experts_by_layer, shapes, layout="runs", shards=1, extra=()):
    """experts_by_layer: {layer: {e: mats}}. Experts are dealt round-robin over `shards` files,
    each expert whole in one file; `extra` tensors go first into shard 0."""
    os.makedirs(d, exist_ok=True)
    files = [list(extra)] + [[] for _ in range(shards - 1)]
    k = 0
    for L in sorted(experts_by_layer):
        for e in sorted(experts_by_layer[L]):
            files[k % shards] += expert_tensors(L, e, experts_by_layer[L][e], shapes, layout)
            k += 1
    for i, ts in enumerate(files):
        write_shard(os.path.join(d, f"model-{i + 1:05d}-of-{shards:05d}.safetensors"), ts)
