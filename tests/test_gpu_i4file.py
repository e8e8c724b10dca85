"""The int4 expert container on the GPU (include/glm53f_i4file.h): this library's writer, which
quantises on the device, against the reference's writer (src/io/glm53f_i4file.c in oracle/_ref,
the reference's CPU quantiser), byte for byte; and the HBM cache in int4 mode reading a layer's
experts from the container (glm53f_i4_dir set) against quantising them on the way in: the same
slot bytes, so the drop-in's outputs are bit-identical."""
import ctypes as C
import filecmp
import os

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
from ckpt_write import write_layers
from glm53h import check
from test_gpu_ckpt import moe_w
from test_gpu_parity import cfg_struct, same, say
import oracle_lib as O

pytestmark = pytest.mark.gpu
NL = 2


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


def ref_writer(ck, out, sp, layer):
    R = O.ref()
    R.ref_i4_write.restype = C.c_int
    R.ref_i4_write.argtypes = [C.c_char_p] + [C.c_int] * 7 + [C.c_char_p]
    return R.ref_i4_write(ck.encode(), sp.E, sp.I, sp.NE, sp.br, sp.bc, NL, layer, out.encode())


def test_container_writer_and_cache(L, tmp_path):
    sps = [S.spec(1, layer=Ly) for Ly in range(NL)]
    sp = sps[0]
    c = dict(E=sp.E, I=sp.I, NE=sp.NE, K=sp.K, routed_scale=sp.routed_scale, norm_topk=sp.norm_topk,
             limit=sp.limit, br=sp.br, bc=sp.bc)
    ex = {Ly: {e: S.expert_host(sps[Ly], e) for e in range(sp.NE)} for Ly in range(NL)}
    ck, ref_d, our_d = (str(tmp_path / n) for n in ("ckpt", "i4ref", "i4ours"))
    os.makedirs(ref_d)
    os.makedirs(our_d)
    say("writing a config-1 checkpoint of", NL, "layers")
    write_layers(ck, ex, [(sp.I, sp.E), (sp.I, sp.E), (sp.E, sp.I)], "runs", 2)
    cf = cfg_struct(c)
    cf.n_layers = NL
    st = glm53h.Glm53fSt()
    assert L.g53h_st_open(C.byref(st), ck.encode(), 1) == 0
    dir_var = C.c_char_p.in_dll(L, "glm53f_i4_dir")
    try:
        say("the containers: the reference's writer and this library's")
        for Ly in range(NL):
            assert ref_writer(ck, ref_d, sp, Ly) == 0
            assert L.glm53f_i4file_write_layer(C.byref(st), C.byref(cf), Ly, our_d.encode()) == 0
            assert L.glm53f_i4file_write_layer(C.byref(st), C.byref(cf), Ly, our_d.encode()) == 1   # complete: skipped
            name = f"layer-{Ly:02d}.i4"
            assert filecmp.cmp(os.path.join(ref_d, name), os.path.join(our_d, name), shallow=False)
            assert L.glm53f_i4file_verify_layer(C.byref(st), C.byref(cf), Ly, our_d.encode()) == 0

        R = [(S.router_host(s_), S.bias_host(s_)) for s_ in sps]
        sh = S.expert_host(sp, "shared")
        xs = [np.ascontiguousarray(S.x_host(sps[Ly], 3, batch=7), np.float32) for Ly in range(NL)]

        def run(dir_bytes):
            dir_var.value = dir_bytes
            cache = glm53h.Glm53fCache()
            probe = glm53h.Glm53fCache()
            assert L.glm53f_cache_init(C.byref(probe), C.byref(st), C.byref(cf), 1 << 30, 0, 1) == 0
            sb = probe.slot_bytes
            L.glm53f_cache_free(C.byref(probe))
            assert L.glm53f_cache_init(C.byref(cache), C.byref(st), C.byref(cf), sb * 12, 2, 1) == 0
            outs = []
            try:
                layers = cache.i4_layers
                for tok in range(3):
                    for Ly in range(NL):
                        w = moe_w(cache.src, R[Ly][0], R[Ly][1], sh, c, Ly)
                        o = np.zeros((1, sp.E), np.float32)
                        L.glm53f_moe(o.ctypes.data, xs[Ly][tok:tok + 1].ctypes.data, C.byref(w), C.byref(cf), 1, None)
                        outs.append(o[0])
                check(L.glm53f_cache_sync(C.byref(cache)), "sync")
                assert cache.misses > 0
                return np.asarray(outs), layers, cache.bytes_read, cache.misses, sb
            finally:
                L.glm53f_cache_free(C.byref(cache))
                dir_var.value = None

        say("int4 cache, quantised on the way in")
        want, l0, _, _, _ = run(None)
        say("int4 cache, read from the containers")
        got, l1, nread, misses, sb = run(our_d.encode())
        assert l0 == 0 and l1 == NL
        assert same(got, want)
        assert nread == misses * sb                      # one container read of a whole slot per miss
    finally:
        dir_var.value = None
        L.g53h_st_close(C.byref(st))
        L.glm53f_forget_host_weights()
