"""The expert cache reading the checkpoint (glm53f_cache_init over a Glm53fSt, the
reference's entry point, src/cache/glm53f_cache.h:99-100): experts go from safetensors shards
through pinned staging into HBM slots, and the drop-in MoE layer on those slots must give the
reference's outputs bit for bit. Two checkpoints: the reference's own glm_tiny fixture (4x4
blocks, its golden layer outputs), and a written config-1 checkpoint of several layers, with a
budget far below the working set so reads, evictions and prefetch all happen."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
import oracle_lib as O
from ckpt_write import write_layers
from glm53h import check
from test_gpu_parity import GOLD, HostSrc, cfg_struct, fmat, same, say

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import tinyst  # noqa: E402

pytestmark = pytest.mark.gpu
TINY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "glm_tiny")


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


def moe_w(src, W, b, sh, c, layer, nxt=None, prefetch_n=0):
    w = glm53h.Glm53fMoeW()
    w.gate, w.bias = W.ctypes.data, b.ctypes.data
    (gw, gs), (uw, us), (dw, ds) = sh
    w.sh_gate = fmat(gw, gs, c["I"], c["E"], c["br"], c["bc"])
    w.sh_up = fmat(uw, us, c["I"], c["E"], c["br"], c["bc"])
    w.sh_down = fmat(dw, ds, c["E"], c["I"], c["br"], c["bc"])
    w.src = C.pointer(src)
    w.layer, w.prefetch_n = layer, prefetch_n
    if nxt is not None:
        w.next_gate, w.next_bias = nxt[0].ctypes.data, nxt[1].ctypes.data
    return w


def open_cache(L, d, cf, slots, n_io):
    st = glm53h.Glm53fSt()
    assert L.g53h_st_open(C.byref(st), d.encode(), 1) == 0
    c = glm53h.Glm53fCache()
    probe = glm53h.Glm53fCache()
    assert L.glm53f_cache_init(C.byref(probe), C.byref(st), C.byref(cf), 1 << 30, 0, 0) == 0
    sb = probe.slot_bytes
    L.glm53f_cache_free(C.byref(probe))
    assert L.glm53f_cache_init(C.byref(c), C.byref(st), C.byref(cf), sb * slots, n_io, 0) == 0
    assert c.nslot == slots and c.st is not None and c.arena and c.i4 == 0
    assert L.g53h_cache_is(C.byref(c.src)) == 1
    return st, c


def test_cache_from_glm_tiny_checkpoint(L):
    """The reference's fixture checkpoint: every MoE layer's golden output (compiled
    reference), with the experts read from the file by the cache."""
    t, cfg = tinyst.load(), tinyst.config()
    cf = cfg_struct(cfg)
    cf.n_layers = 5
    cf.is_dense[0] = 1
    for slots, n_io in ((cfg["K"] + 1, 0), (12, 2)):
        st, c = open_cache(L, TINY, cf, slots, n_io)
        try:
            layers = cfg["moe_layers"]
            ws = {Ly: tinyst.layer(t, Ly) for Ly in layers}
            for i, Ly in enumerate(layers):
                W, b, _, sh = ws[Ly]
                nxt = ws[layers[i + 1]][:2] if i + 1 < len(layers) else None
                w = moe_w(c.src, W, b, sh, cfg, Ly, nxt, prefetch_n=4 if n_io else 0)
                x = np.ascontiguousarray(GOLD[f"tiny{Ly}_x"], np.float32)
                out = np.zeros_like(x)
                say("glm_tiny from the checkpoint: layer", Ly, "slots", slots, "prefetch", n_io)
                L.glm53f_moe(out.ctypes.data, x.ctypes.data, C.byref(w), C.byref(cf), x.shape[0], None)
                assert same(out, GOLD[f"tiny{Ly}_out"])
                for tok in range(2):                               # decode, one token at a time
                    o1 = np.zeros((1, cfg["E"]), np.float32)
                    L.glm53f_moe(o1.ctypes.data, x[tok:tok + 1].ctypes.data, C.byref(w), C.byref(cf), 1, None)
                    assert same(o1, GOLD[f"tiny{Ly}_out"][tok:tok + 1])
            check(L.glm53f_cache_sync(C.byref(c)), "sync")
            assert c.misses + c.prefetch_reads + c.bg_reads > 0 and c.bytes_read + c.bg_bytes > 0
            if slots < 12:
                assert c.evictions > 0
        finally:
            L.glm53f_cache_free(C.byref(c))
            L.g53h_st_close(C.byref(st))
    L.glm53f_forget_host_weights()


def test_cache_from_written_checkpoint_many_layers(L, tmp_path):
    """Six layers of 16 config-1 experts in two shards (weights and scales as runs); 12 slots for
    96 experts. Every output equals the host-memory path's; sampled ones equal the oracle's."""
    NL, T = 6, 3
    sps = [S.spec(1, layer=Ly) for Ly in range(NL)]
    sp = sps[0]
    c = dict(E=sp.E, I=sp.I, NE=sp.NE, K=sp.K, routed_scale=sp.routed_scale, norm_topk=sp.norm_topk,
             limit=sp.limit, br=sp.br, bc=sp.bc)
    ex = {Ly: {e: S.expert_host(sps[Ly], e) for e in range(sp.NE)} for Ly in range(NL)}
    d = str(tmp_path / "ckpt")
    say("writing a", NL, "layer checkpoint")
    write_layers(d, ex, [(sp.I, sp.E), (sp.I, sp.E), (sp.E, sp.I)], "runs", 2)
    cf = cfg_struct(c)
    cf.n_layers = NL
    R = [(S.router_host(s_), S.bias_host(s_)) for s_ in sps]
    sh = S.expert_host(sp, "shared")
    xs = [np.ascontiguousarray(S.x_host(sps[Ly], T, batch=9), np.float32) for Ly in range(NL)]

    def run(src_of, pf):
        outs = {}
        for tok in range(T):
            for Ly in range(NL):
                nxt = R[Ly + 1] if Ly + 1 < NL else None
                w = moe_w(src_of(Ly), R[Ly][0], R[Ly][1], sh, c, Ly, nxt, pf)
                o = np.zeros((1, sp.E), np.float32)
                L.glm53f_moe(o.ctypes.data, xs[Ly][tok:tok + 1].ctypes.data, C.byref(w), C.byref(cf), 1, None)
                outs[(tok, Ly)] = o[0]
        return outs

    hosts = [HostSrc(cf, ex[Ly]) for Ly in range(NL)]
    want = run(lambda Ly: hosts[Ly].src, 0)
    st, cache = open_cache(L, d, cf, 12, 2)
    try:
        say("six layers through the cache from the checkpoint")
        got = run(lambda Ly: cache.src, 6)
        check(L.glm53f_cache_sync(C.byref(cache)), "sync")
        assert all(same(got[k], want[k]) for k in want)
        assert cache.misses > 0 and cache.evictions > 0 and cache.bg_reads > 0
        assert cache.hits + cache.misses == T * NL * sp.K
        for tok, Ly in ((0, 0), (2, 5)):
            o, _, _ = O.moe(O.oracle(), xs[Ly][tok:tok + 1], sps[Ly], R[Ly][0], R[Ly][1], ex[Ly], sh)
            assert same(got[(tok, Ly)], o[0])
    finally:
        L.glm53f_cache_free(C.byref(cache))
        L.g53h_st_close(C.byref(st))
        L.glm53f_forget_host_weights()
