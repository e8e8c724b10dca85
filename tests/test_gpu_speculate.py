"""GPU parity of the pieces of the drop-in's speculative cached decode: the next layer's router
scores requested of the decode launch (g53h_decode_next), and the one launch that publishes
the routing, the next layer's top-n prediction, the error words and the output into the host
mailbox (g53h_decode_publish).

Bar: the routing and the output bit-exact against the C oracle (src/core/glm53f_ops.c:945-976,
1329-1340); the prediction index for index against the oracle's route_topn
(src/core/glm53f_ops.c:1021-1042). Both ways of computing the next scores are covered: by the
spare waves of the one-launch decode kernels (octet-tiled and MFMA-tiled), and by a launch of
their own when no decode launch took the request."""
import ctypes as C

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
import oracle_lib as O
from glm53h import DevBuf, check
from test_gpu_parity import same, say
from test_gpu_predict import topn_oracle
from test_gpu_grouped import within

pytestmark = pytest.mark.gpu
SLOT, ROUTE_OFF, OUT_OFF = 7, 8192, 16384      # a mailbox slot and areas the drop-in does not use
NERR = 3


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


@pytest.fixture(scope="module")
def tiled(L):
    say("building the config-2 layer, octet-tiled")
    return S.DeviceLayer.build(S.spec(2), tiled=True)


def mailbox_words(L, off, n, dtype):
    base = L.g53h_mailbox()
    return np.frombuffer(C.string_at(base + off, 4 * n), dtype).copy()


def publish_round(L, layer, x, Wn, bn, n, seq, out_off=OUT_OFF):
    sp = layer.sp
    xd = DevBuf.from_array(np.ascontiguousarray(x[0]))
    gate = DevBuf.from_array((np.ascontiguousarray(Wn, np.float32).view(np.uint32) >> 16).astype(np.uint16))
    bd = DevBuf.from_array(np.ascontiguousarray(bn, np.float32))
    out, idx, w, pred = DevBuf(sp.E * 4), DevBuf(sp.K * 4), DevBuf(sp.K * 4), DevBuf(max(n, 1) * 4)
    check(L.g53h_decode_next(xd.ptr, gate.ptr, 1, bd.ptr, sp.NE, sp.E), "g53h_decode_next")
    layer.forward(out, xd, 1, idx, w)
    check(L.g53h_decode_publish(SLOT, seq, ROUTE_OFF, idx.ptr, sp.K, pred.ptr, n, sp.NE, out_off, out.ptr, sp.E * 4),
          "g53h_decode_publish")
    check(L.g53h_mailbox_wait(SLOT, seq), "mailbox wait")
    r = mailbox_words(L, ROUTE_OFF, sp.K + 1 + n, np.int32)
    errs = mailbox_words(L, out_off, NERR, np.int32)
    o = mailbox_words(L, out_off + 4 * NERR, sp.E, np.float32)
    glm53h.sync()
    assert np.array_equal(o.view(np.uint32), out.download(np.float32).view(np.uint32))
    assert np.array_equal(r[:sp.K], idx.download(np.int32))
    return r[:sp.K], r[sp.K], r[sp.K + 1:], errs, o, w.download(np.float32)


def next_router(sp):
    nsp = S.spec(2, layer=1)
    return S.router_host(nsp), S.bias_host(nsp)


def test_next_scores_in_the_tiled_decode(L, tiled):
    sp = tiled.sp
    Wn, bn = next_router(sp)
    x = S.x_host(sp, 3, batch=4)
    for t in range(3):
        say("tiled decode + next scores + publish, token", t)
        # the output 16-byte aligned in the mailbox (16-byte stores) on the last token
        ids, nan, pred, errs, out, w = publish_round(L, tiled, x[t:t + 1], Wn, bn, 6, 900 + t,
                                                     OUT_OFF + 4 if t == 2 else OUT_OFF)
        assert nan == 0 and not errs[:3].any()
        assert np.array_equal(pred, topn_oracle(x[t:t + 1], Wn, bn, 6)[0])
        mats = {int(e): tiled.fetch_expert(int(e)) for e in ids}
        want, wi, ww = O.moe(O.oracle(), x[t:t + 1], sp, tiled.router_f32, tiled.bias_f32, mats,
                             tiled.fetch_expert("shared"))
        assert np.array_equal(ids, wi[0]) and same(w, ww[0]) and same(out, want[0])


def test_next_scores_in_the_mfma_decode(L):
    """The MFMA-tiled decode's spare waves compute the requested scores."""
    sp = S.spec(2)
    say("building the config-2 layer, MFMA-tiled")
    m = S.DeviceLayer.build(sp, mfma=True)
    Wn, bn = next_router(sp)
    x = S.x_host(sp, 1, batch=5)
    ids, nan, pred, errs, out, w = publish_round(L, m, x, Wn, bn, 16, 950)
    assert nan == 0 and not errs[:3].any()
    assert np.array_equal(pred, topn_oracle(x, Wn, bn, 16)[0])
    mats = {int(e): m.fetch_expert(int(e)) for e in ids}
    want, wi, _ = O.moe(O.oracle(), x, sp, m.router_f32, m.bias_f32, mats, m.fetch_expert("shared"))
    assert np.array_equal(ids, wi[0])
    within(out[None], want, "mfma decode through the publish launch")


def test_publish_without_prediction(L, tiled):
    sp = tiled.sp
    x = S.x_host(sp, 1, batch=6)
    xd = DevBuf.from_array(np.ascontiguousarray(x[0]))
    out, idx, w = DevBuf(sp.E * 4), DevBuf(sp.K * 4), DevBuf(sp.K * 4)
    tiled.forward(out, xd, 1, idx, w)
    check(L.g53h_decode_publish(SLOT, 990, ROUTE_OFF, idx.ptr, sp.K, None, 0, sp.NE, OUT_OFF, out.ptr, sp.E * 4),
          "publish")
    check(L.g53h_mailbox_wait(SLOT, 990), "wait")
    r = mailbox_words(L, ROUTE_OFF, sp.K + 1, np.int32)
    glm53h.sync()
    assert np.array_equal(r[:sp.K], idx.download(np.int32)) and r[sp.K] == 0
    # a request the publish cannot serve (other expert count) is an error, not a wrong prediction
    Wn, bn = next_router(sp)
    gate = DevBuf.from_array((np.ascontiguousarray(Wn, np.float32).view(np.uint32) >> 16).astype(np.uint16))
    bd = DevBuf.from_array(bn)
    pred = DevBuf(64)
    check(L.g53h_decode_next(xd.ptr, gate.ptr, 1, bd.ptr, sp.NE, sp.E), "arm")
    assert L.g53h_decode_publish(SLOT, 991, ROUTE_OFF, idx.ptr, sp.K, pred.ptr, 4, sp.NE - 1, OUT_OFF, out.ptr,
                                 sp.E * 4) != 0
    glm53h.sync()


def test_next_scores_by_their_own_launch(L, tiled):
    """A request that no decode launch took: the publish launch computes the scores."""
    sp = tiled.sp
    Wn, bn = next_router(sp)
    x = S.x_host(sp, 1, batch=8)
    xd = DevBuf.from_array(np.ascontiguousarray(x[0]))
    out, idx, w = DevBuf(sp.E * 4), DevBuf(sp.K * 4), DevBuf(sp.K * 4)
    tiled.forward(out, xd, 1, idx, w)
    gate = DevBuf.from_array((np.ascontiguousarray(Wn, np.float32).view(np.uint32) >> 16).astype(np.uint16))
    bd = DevBuf.from_array(np.ascontiguousarray(bn, np.float32))
    pred = DevBuf(6 * 4)
    say("next scores armed after the decode: the publish launch computes them")
    check(L.g53h_decode_next(xd.ptr, gate.ptr, 1, bd.ptr, sp.NE, sp.E), "g53h_decode_next")
    check(L.g53h_decode_publish(SLOT, 995, ROUTE_OFF, idx.ptr, sp.K, pred.ptr, 6, sp.NE, OUT_OFF, out.ptr, sp.E * 4),
          "g53h_decode_publish")
    check(L.g53h_mailbox_wait(SLOT, 995), "mailbox wait")
    r = mailbox_words(L, ROUTE_OFF, sp.K + 1 + 6, np.int32)
    glm53h.sync()
    assert np.array_equal(r[sp.K + 1:], topn_oracle(x, Wn, bn, 6)[0])
