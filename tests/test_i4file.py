"""The int4 expert container (include/glm53f_i4file.h, host/g53h_i4file.c) on the CPU, against
files the reference's own writer makes (src/io/glm53f_i4file.c, compiled into oracle/_ref, which
quantises with the reference's glm53f_i4_from_f8): this library accepts them for the checkpoint
they came from (the header's fingerprint recomputed from this library's reader), verifies their
CRCs, finds a flipped byte, and refuses an incomplete file, another geometry and the same
experts laid out differently in the shards."""
import ctypes as C
import os

import numpy as np

import glm53h
import oracle_lib as O
from ckpt_write import write_layers

E, I, NE, NL = 256, 128, 5, 2


def make_ckpt(d, layout="runs", seed=3):
    rng = np.random.default_rng(seed)
    shapes = [(I, E), (I, E), (E, I)]

    def mats():
        out = []
        for r, c in shapes:
            w = rng.integers(0, 256, r * c).astype(np.uint8)
            w[(w & 0x7f) == 0x7f] ^= 1                       # no NaN codes
            s = rng.uniform(1e-3, 1e-1, ((r + 127) // 128) * ((c + 127) // 128)).astype(np.float32)
            out.append((w, s))
        return out

    write_layers(d, {L: {e: mats() for e in range(NE)} for L in range(NL)}, shapes, layout)


def cfg(n_experts=NE):
    cf = glm53h.Glm53fCfg()
    cf.hidden, cf.moe_inter, cf.n_experts, cf.fp8_block_r, cf.fp8_block_c, cf.n_layers = E, I, n_experts, 128, 128, NL
    return cf


def ref_write(ckpt, out, layer):
    R = O.ref()
    R.ref_i4_write.restype = C.c_int
    R.ref_i4_write.argtypes = [C.c_char_p] + [C.c_int] * 7 + [C.c_char_p]
    return R.ref_i4_write(ckpt.encode(), E, I, NE, 128, 128, NL, layer, out.encode())


def ours(ckpt):
    L = glm53h.lib()
    st = glm53h.Glm53fSt()
    assert L.g53h_st_open(C.byref(st), ckpt.encode(), 0) == 0
    return L, st


def opened(L, st, cf, layer, d):
    fd = L.glm53f_i4file_open_layer(C.byref(st), C.byref(cf), layer, d.encode())
    if fd >= 0:
        os.close(fd)
    return fd


def test_reference_container_accepted_and_verified(tmp_path):
    ck, out = str(tmp_path / "ckpt"), str(tmp_path / "i4")
    os.makedirs(out)
    make_ckpt(ck)
    for layer in range(NL):
        assert ref_write(ck, out, layer) == 0
    L, st = ours(ck)
    try:
        cf = cfg()
        for layer in range(NL):
            assert opened(L, st, cf, layer, out) >= 0
            assert L.glm53f_i4file_verify_layer(C.byref(st), C.byref(cf), layer, out.encode()) == 0
        # the file is header + NE slots of the reference's int4 layout
        sz = os.path.getsize(os.path.join(out, "layer-00.i4"))
        assert (sz - 4096) % NE == 0 and (sz - 4096) // NE % 4096 == 0
        slot = (sz - 4096) // NE
        # 3 x (levels rows x cols / 2, steps rows x cols / 64 x 4 B), 64-byte aligned, 4 KiB rounded
        assert slot == (3 * I * E // 2 + 3 * I * E // 64 * 4 + 4095) // 4096 * 4096 == 57344
        # a flipped byte in expert 3 is found by its CRC
        p = os.path.join(out, "layer-01.i4")
        with open(p, "r+b") as f:
            f.seek(4096 + 3 * slot + 1000)
            b = f.read(1)
            f.seek(4096 + 3 * slot + 1000)
            f.write(bytes([b[0] ^ 0x10]))
        assert L.glm53f_i4file_verify_layer(C.byref(st), C.byref(cf), 1, out.encode()) == 1
        # no completion mark: refused
        with open(p, "r+b") as f:
            f.seek(40)
            f.write((0).to_bytes(4, "little"))
        assert opened(L, st, cf, 1, out) == -2
        # another geometry, a missing layer
        assert opened(L, st, cfg(NE + 1), 0, out) == -2
        assert opened(L, st, cf, 0, str(tmp_path)) == -1
    finally:
        L.g53h_st_close(C.byref(st))


def test_container_refused_for_another_shard_layout(tmp_path):
    """The same experts written with weights and scales interleaved: their tensors no longer form
    two runs, so the fingerprint differs and the reference's file for the run layout is refused
    (and one written from the interleaved checkpoint is accepted)."""
    runs, inter, out, out2 = (str(tmp_path / n) for n in ("runs", "inter", "i4", "i4b"))
    os.makedirs(out)
    os.makedirs(out2)
    make_ckpt(runs, "runs")
    make_ckpt(inter, "interleaved")
    assert ref_write(runs, out, 0) == 0
    assert ref_write(inter, out2, 0) == 0
    L, st = ours(inter)
    try:
        assert opened(L, st, cfg(), 0, out) == -2
        assert opened(L, st, cfg(), 0, out2) >= 0
    finally:
        L.g53h_st_close(C.byref(st))
    with open(os.path.join(out, "layer-00.i4"), "rb") as a, open(os.path.join(out2, "layer-00.i4"), "rb") as b:
        ha, hb = a.read(4096), b.read(4096)
        assert ha[:24] == hb[:24] and ha[32:40] != hb[32:40]   # same geometry, another fingerprint
        assert a.read() == b.read()                              # the same quantised experts
