"""g53h_moe_decode_noalloc (the decode entry point that allocates nothing) against g53h_moe at
T = 1 on the same layer, bit for bit, on two calls in a row, the second on a smaller layer
(fewer experts, smaller top-k); and its rejections."""
import ctypes as C

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
from glm53h import DevBuf, check
from test_gpu_parity import same, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


def both(L, layer, x):
    """(out, idx, w) from g53h_moe and from g53h_moe_decode_noalloc."""
    sp = layer.sp
    xd = DevBuf.from_array(np.ascontiguousarray(x, np.float32))
    res = []
    for noalloc in (False, True):
        out, idd, wd = DevBuf(sp.E * 4), DevBuf(sp.K * 4), DevBuf(sp.K * 4)
        if noalloc:
            check(L.g53h_moe_decode_noalloc(out.ptr, xd.ptr, C.byref(layer.layer), idd.ptr, wd.ptr),
                  "g53h_moe_decode_noalloc")
        else:
            check(L.g53h_moe(out.ptr, xd.ptr, 1, C.byref(layer.layer), idd.ptr, wd.ptr), "g53h_moe")
        glm53h.sync()
        assert L.g53h_decode_errors() == 0
        res.append((out.download(np.float32), idd.download(np.int32), wd.download(np.float32)))
    return res


def test_noalloc_matches_g53h_moe(L):
    assert L.g53h_set_fused_decode(1) == 1
    big = S.DeviceLayer.build(S.spec(2), tiled=True)
    small = S.DeviceLayer.build(S.spec(2, NE=64, K=4, shared=False, seed=13), tiled=True)
    for layer, batch in ((big, 50), (small, 51), (big, 52)):
        sp = layer.sp
        say("no-alloc decode, NE", sp.NE, "K", sp.K)
        (o1, i1, w1), (o2, i2, w2) = both(L, layer, S.x_host(sp, 1, batch=batch))
        assert np.array_equal(i1, i2) and same(w1, w2) and same(o1, o2)


def test_noalloc_rejections(L):
    rm = S.DeviceLayer.build(S.spec(2, NE=16, K=4, seed=14))           # row-major experts
    sp = rm.sp
    xd, out = DevBuf(sp.E * 4), DevBuf(sp.E * 4)
    assert L.g53h_moe_decode_noalloc(out.ptr, xd.ptr, C.byref(rm.layer), None, None) != 0
    assert b"octet-tiled" in L.g53h_error()
    lay = glm53h.G53hMoeLayer.from_buffer_copy(bytes(rm.layer))
    lay.tiled, lay.n_experts = 1, 1025
    assert L.g53h_moe_decode_noalloc(out.ptr, xd.ptr, C.byref(lay), None, None) != 0
    assert b"above the limit of 1024" in L.g53h_error()
    lay.n_experts, lay.topk = 16, 16
    assert L.g53h_moe_decode_noalloc(out.ptr, xd.ptr, C.byref(lay), None, None) != 0
    assert b"above the limit of 15" in L.g53h_error()
