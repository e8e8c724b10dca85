"""The checkpoint side of the expert cache, on the CPU: this library's safetensors reader
(g53h_st_open) against the reference's (src/io/glm53f_st.c, compiled into oracle/_ref) on the
reference's glm_tiny fixture and on written checkpoints, and the expert staging read
(g53h_st_read_expert) against the reference's loader (src/io/glm53f_load.c:85-208) and the
bytes written: weights as one run and scales as another, interleaved tensors, tensors in
reverse order, several shards, and O_DIRECT descriptors where the filesystem has them."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
import oracle_lib as O
from ckpt_write import write_layers

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import tinyst  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
TINY = os.path.join(HERE, "golden", "glm_tiny")


def ours_table(d, direct=0):
    L = glm53h.lib()
    st = glm53h.Glm53fSt()
    assert L.g53h_st_open(C.byref(st), d.encode(), direct) == 0
    rows, names = [], []
    for i in range(st.nt):
        t = st.t[i]
        rows.append([t.shard, t.dtype, t.ndim, t.shape[0] if t.ndim > 0 else 0, t.shape[1] if t.ndim > 1 else 0,
                     t.off, t.nbytes])
        names.append(t.name.decode())
    return st, np.array(rows, np.int64), names


def ref_table(d):
    R = O.ref()
    R.ref_st_table.restype = C.c_int
    R.ref_st_table.argtypes = [C.c_char_p, C.c_void_p, C.c_int, C.c_char_p, C.c_int]
    meta = np.zeros((100000, 7), np.int64)
    names = C.create_string_buffer(1 << 22)
    n = R.ref_st_table(d.encode(), meta.ctypes.data, 100000, names, 1 << 22)
    assert n >= 0
    return meta[:n], names.value.decode().split("\n")[:n]


def cfg_of(E, I, NE, br=128, bc=128, n_layers=2):
    cf = glm53h.Glm53fCfg()
    cf.hidden, cf.moe_inter, cf.n_experts, cf.fp8_block_r, cf.fp8_block_c, cf.n_layers = E, I, NE, br, bc, n_layers
    return cf


def read_expert(st, cf, layer, e):
    """g53h_st_read_expert -> gate, up, down codes then scales, as bytes (None on failure)."""
    L = glm53h.lib()
    cap = L.g53h_st_expert_bytes(C.byref(cf))
    buf = (C.c_uint8 * cap)()
    q = glm53h.Glm53fExpertQ()
    if L.g53h_st_read_expert(C.byref(st), C.byref(cf), layer, e, buf, cap, C.byref(q)) != 0:
        return None
    ms = [q.gate, q.up, q.down]
    out = b"".join(C.string_at(m.w, m.rows * m.cols) for m in ms)
    return out + b"".join(C.string_at(m.s, ((m.rows + m.br - 1) // m.br) * m.scols * 4) for m in ms)


def ref_expert(d, cf, layer, e):
    R = O.ref()
    R.ref_expert_read.restype = C.c_longlong
    R.ref_expert_read.argtypes = [C.c_char_p] + [C.c_int] * 7 + [C.c_void_p, C.c_longlong]
    out = np.zeros(64 << 20, np.uint8)
    n = R.ref_expert_read(d.encode(), cf.hidden, cf.moe_inter, cf.n_experts, cf.fp8_block_r, cf.fp8_block_c,
                          layer, e, out.ctypes.data, out.nbytes)
    return None if n < 0 else out[:n].tobytes()


def expected(mats):
    return b"".join(np.asarray(w, np.uint8).tobytes() for w, _ in mats) + \
        b"".join(np.asarray(s, np.float32).tobytes() for _, s in mats)


@pytest.mark.skipif(not O.have_ref(), reason="reference not built")
def test_reader_matches_reference_on_glm_tiny():
    st, rows, names = ours_table(TINY)
    try:
        want, wnames = ref_table(TINY)
        assert names == wnames and np.array_equal(rows, want)
        assert st.nshard == 1 and st.nt == len(names) > 100
    finally:
        glm53h.lib().g53h_st_close(C.byref(st))


@pytest.mark.skipif(not O.have_ref(), reason="reference not built")
def test_glm_tiny_expert_bytes_match_reference_loader():
    t, c = tinyst.load(), tinyst.config()
    cf = cfg_of(c["E"], c["I"], c["NE"], c["br"], c["bc"], n_layers=5)
    st, _, _ = ours_table(TINY)
    try:
        for L in c["moe_layers"]:
            _, _, ex, _ = tinyst.layer(t, L)
            for e in (0, c["NE"] - 1):
                got = read_expert(st, cf, L, e)
                assert got == ref_expert(TINY, cf, L, e) == expected(ex[e])
    finally:
        glm53h.lib().g53h_st_close(C.byref(st))


@pytest.mark.parametrize("layout,shards,direct", [("runs", 1, 0), ("runs", 3, 1), ("interleaved", 2, 0),
                                                  ("reversed", 1, 1)])
def test_written_checkpoint_layouts(tmp_path, layout, shards, direct):
    sp = S.spec(1)
    NE = 4
    shapes = [(sp.I, sp.E), (sp.I, sp.E), (sp.E, sp.I)]
    ex = {L: {e: S.expert_host(S.spec(1, layer=L), e) for e in range(NE)} for L in (0, 1)}
    router = np.zeros((NE, sp.E), np.uint16)
    d = str(tmp_path / "ckpt")
    write_layers(d, ex, shapes, layout, shards, extra=[("model.language_model.layers.0.mlp.gate.weight", router)])
    cf = cfg_of(sp.E, sp.I, NE)
    st, rows, names = ours_table(d, direct)
    try:
        assert st.nshard == shards and len(names) == 1 + 2 * NE * 6
        if O.have_ref():
            want, wnames = ref_table(d)
            assert names == wnames and np.array_equal(rows, want)
        for L in (0, 1):
            for e in range(NE):
                got = read_expert(st, cf, L, e)
                assert got == expected(ex[L][e]), (L, e)
                if O.have_ref() and e in (0, NE - 1):
                    assert got == ref_expert(d, cf, L, e)
        assert read_expert(st, cf, 2, 0) is None and read_expert(st, cf, 0, NE) is None
    finally:
        glm53h.lib().g53h_st_close(C.byref(st))


def test_malformed_experts_are_refused(tmp_path):
    sp = S.spec(1)
    shapes = [(sp.I, sp.E), (sp.I, sp.E), (sp.E, sp.I)]
    good = S.expert_host(sp, 0)
    (gw, gs), (uw, us), (dw, ds) = good
    bad_shape = [(gw, gs), (uw, us), (dw[: sp.E * sp.I // 2], ds)]
    d = str(tmp_path / "bad")
    write_layers(d, {0: {0: good}}, shapes)
    # expert 1: down has half its rows; expert 2: no scales for up
    from ckpt_write import expert_tensors, write_shard
    t1 = expert_tensors(0, 1, good, shapes, "runs")
    t1[2] = (t1[2][0], np.asarray(dw, np.uint8).reshape(sp.E, sp.I)[: sp.E // 2])
    t2 = [t for t in expert_tensors(0, 2, good, shapes, "runs") if "up_proj.weight_scale_inv" not in t[0]]
    write_shard(os.path.join(d, "model-00002-of-00002.safetensors"), t1 + t2)
    st, _, _ = ours_table(d)
    cf = cfg_of(sp.E, sp.I, 4)
    try:
        assert read_expert(st, cf, 0, 0) == expected(good)
        assert read_expert(st, cf, 0, 1) is None
        assert read_expert(st, cf, 0, 2) is None
    finally:
        glm53h.lib().g53h_st_close(C.byref(st))
    (tmp_path / "trunc").mkdir()
    with open(tmp_path / "trunc" / "x.safetensors", "wb") as f:
        f.write((10 ** 6).to_bytes(8, "little") + b"{}")
    st = glm53h.Glm53fSt()
    assert glm53h.lib().g53h_st_open(C.byref(st), str(tmp_path / "trunc").encode(), 0) == -1
    del bad_shape
