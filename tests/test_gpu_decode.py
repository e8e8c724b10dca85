"""GPU parity of the one-launch decode kernel (k_dec_layer, T = 1) beyond the released
configuration: other expert counts (the 16-keys-per-lane top-k for more than 320 experts),
other top-k, no shared expert, and experts that are absent or have an unusable descriptor.

Bar: bit-exact routing and outputs against the C oracle (the decode kernel reproduces the
reference's arithmetic step by step), for the same seeded inputs."""
import ctypes as C

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
import oracle_lib as O
from glm53h import DevBuf
from test_gpu_parity import run_layer, same, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


def oracle_check(layer, x, out, idx, w, drop=()):
    sp = layer.sp
    mats = {int(e): layer.fetch_expert(int(e)) for e in idx[0] if int(e) not in drop}
    sh = layer.fetch_expert("shared") if sp.shared else None
    want, wi, ww = O.moe(O.oracle(), x, sp, layer.router_f32, layer.bias_f32, mats, sh)
    assert np.array_equal(idx, wi) and same(w, ww)
    assert same(out, want)


@pytest.mark.parametrize("NE,K,shared,norm", [(512, 4, False, 1), (288, 15, True, 1), (640, 8, True, 0)])
def test_decode_other_layouts(L, NE, K, shared, norm):
    sp = S.spec(2, NE=NE, K=K, shared=shared, norm_topk=norm, seed=11)
    say("decode layout NE", NE, "K", K, "shared", shared, "norm_topk", norm)
    layer = S.DeviceLayer.build(sp)
    assert L.g53h_set_fused_decode(1) == 1
    for t in range(2):
        x = S.x_host(sp, 1, batch=20 + t)
        out, idx, w = run_layer(layer, x, 1)
        assert L.g53h_decode_errors() == 0
        oracle_check(layer, x, out, idx, w)
    del layer


def test_decode_absent_and_unusable_experts(L):
    """A routed expert whose descriptor has no codes contributes zero (the reference's drop
    path); one with unusable blocks is flagged (bit 8) and contributes zero too."""
    sp = S.spec(2, seed=12)
    layer = S.DeviceLayer.build(sp)
    x = S.x_host(sp, 1, batch=30)
    _, idx, _ = run_layer(layer, x, 1)
    gone, bad = int(idx[0][2]), int(idx[0][5])
    say("decode with expert", gone, "absent and", bad, "unusable")
    descs = (glm53h.G53hExpert * (sp.NE + 1)).from_buffer_copy(bytes(layer.experts))
    descs[gone].gate.w = None
    descs[bad].up.bc = 64
    table = DevBuf.from_array(np.frombuffer(bytes(descs), np.uint8))
    lay = glm53h.G53hMoeLayer.from_buffer_copy(bytes(layer.layer))
    lay.experts = table.ptr
    lay.shared = table.ptr + sp.NE * C.sizeof(glm53h.G53hExpert)
    xd = DevBuf.from_array(x)
    out, idd, wd = DevBuf(sp.E * 4), DevBuf(sp.K * 4), DevBuf(sp.K * 4)
    glm53h.check(L.g53h_moe(out.ptr, xd.ptr, 1, C.byref(lay), idd.ptr, wd.ptr), "g53h_moe")
    glm53h.sync()
    assert L.g53h_decode_errors() == 8
    oracle_check(layer, x, out.download(np.float32).reshape(1, sp.E), idd.download(np.int32).reshape(1, sp.K),
                 wd.download(np.float32).reshape(1, sp.K), drop=(gone, bad))
