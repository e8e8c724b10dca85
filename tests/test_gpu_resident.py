"""The drop-in keeps host weights resident in HBM keyed by address, checked against sampled
content: weights rewritten in place at the same address (a caller that frees its weights and
gets the address back for others) are uploaded again, never served stale."""
import numpy as np
import pytest

import glm53h
import glm53h.synth as S
from test_gpu_parity import cfg_struct, dropin_moe, same, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


def test_rewritten_weights_are_reuploaded(L):
    sp, sp2 = S.spec(1), S.spec(1, seed=5)
    cf = cfg_struct(dict(E=sp.E, I=sp.I, NE=sp.NE, K=sp.K, routed_scale=sp.routed_scale, norm_topk=sp.norm_topk,
                         limit=sp.limit, br=sp.br, bc=sp.bc))
    ex = {e: S.expert_host(sp, e) for e in range(sp.NE)}
    W, b = S.router_host(sp).copy(), S.bias_host(sp).copy()
    sh = [tuple(a.copy() for a in m) for m in S.expert_host(sp, "shared")]
    x = S.x_host(sp, 1, batch=3)
    say("drop-in with the first weights")
    first = dropin_moe(cf, W, b, ex, sh, x, forget=False)
    # the same arrays (same addresses) now hold other weights
    W[:] = S.router_host(sp2)
    b[:] = S.bias_host(sp2)
    for (w_, s_), (w2, s2) in zip(sh, S.expert_host(sp2, "shared")):
        w_[:] = w2
        s_[:] = s2
    say("drop-in after rewriting the weights in place")
    second = dropin_moe(cf, W, b, ex, sh, x, forget=False)
    fresh = dropin_moe(cf, W.copy(), b.copy(), ex, [tuple(a.copy() for a in m) for m in sh], x)
    assert same(second, fresh) and not same(second, first)
