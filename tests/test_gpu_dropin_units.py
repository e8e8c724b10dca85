"""GPU parity of the drop-in's unit operations, called as the reference's callers call them
(include/glm53f.h, host pointers): glm53f_mlp (the shared expert / dense MLP, src/core/glm53f_ops.c:
496-511), glm53f_swiglu_clamp (:486-494), glm53f_mm_batch (:376-444, per token as glm53f_mm) on FP8
and int4 matrices. Bar: bit-exact against the oracle."""
import ctypes as C

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
import oracle_lib as O
from test_gpu_parity import cfg_struct, fmat, same, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


def oracle_expert(sp, x, mats):
    """gate, up, SwiGLU, down of one FP8 expert through the oracle, per token."""
    out = []
    for t in range(x.shape[0]):
        (gw, gs), (uw, us), (dw, ds) = mats
        g = O.mm_f8(O.oracle(), x[t], gw, gs, sp.I, sp.E, sp.br, sp.bc)[0]
        u = O.mm_f8(O.oracle(), x[t], uw, us, sp.I, sp.E, sp.br, sp.bc)[0]
        gu = np.concatenate([g, u])
        a = np.empty(sp.I, np.float32)
        O.oracle().or_swiglu(a.ctypes.data, gu.ctypes.data, sp.I, C.c_float(sp.limit))
        out.append(O.mm_f8(O.oracle(), a, dw, ds, sp.E, sp.I, sp.br, sp.bc)[0])
    return np.stack(out)


@pytest.mark.parametrize("config", [1, 2])
def test_dropin_mlp_is_the_oracle_expert(L, config):
    sp = S.spec(config)
    mats = S.expert_host(sp, "shared")
    (gw, gs), (uw, us), (dw, ds) = mats
    gm, um = fmat(gw, gs, sp.I, sp.E, sp.br, sp.bc), fmat(uw, us, sp.I, sp.E, sp.br, sp.bc)
    dm = fmat(dw, ds, sp.E, sp.I, sp.br, sp.bc)
    x = np.ascontiguousarray(S.x_host(sp, 3, batch=6), np.float32)
    want = oracle_expert(sp, x, mats)
    cf = cfg_struct(dict(E=sp.E, I=sp.I, NE=sp.NE, K=sp.K, routed_scale=sp.routed_scale, norm_topk=sp.norm_topk,
                         limit=sp.limit, br=sp.br, bc=sp.bc))
    scratch = np.zeros(L.glm53f_mlp_scratch(C.byref(cf)), np.float32)
    for t in range(3):
        say("glm53f_mlp config", config, "token", t)
        out = np.zeros(sp.E, np.float32)
        xt = np.ascontiguousarray(x[t])
        L.glm53f_mlp(out.ctypes.data, xt.ctypes.data, C.byref(gm), C.byref(um), C.byref(dm), C.c_float(sp.limit),
                     scratch.ctypes.data)
        assert same(out, want[t])
    L.glm53f_forget_host_weights()


def test_dropin_swiglu_clamp(L):
    rng = np.random.default_rng(3)
    for n, limit in [(1, 10.0), (128, 0.5), (2048, 10.0), (777, 3.0)]:
        gu = (rng.standard_normal(2 * n) * 6).astype(np.float32)
        gu[:4 if n >= 2 else 1] = [100.0, -100.0, 0.0, -0.0][:4 if n >= 2 else 1]
        got = np.zeros(n, np.float32)
        L.glm53f_swiglu_clamp(got.ctypes.data, gu.ctypes.data, n, C.c_float(limit))
        want = np.zeros(n, np.float32)
        O.oracle().or_swiglu(want.ctypes.data, gu.ctypes.data, n, C.c_float(limit))
        assert same(got, want), (n, limit)


def test_dropin_mm_batch_fp8_and_int4(L):
    """glm53f_mm_batch on T = 5 inputs equals glm53f_mm per token and the oracle, for an FP8
    matrix with ragged blocks and for an int4 matrix."""
    rng = np.random.default_rng(4)
    rows, cols, br, bc = 300, 1000, 16, 128
    w = rng.integers(0, 256, rows * cols).astype(np.uint8)
    w[(w & 0x7f) == 0x7f] ^= 1
    s = rng.uniform(1e-3, 1e-1, ((rows + br - 1) // br) * ((cols + bc - 1) // bc)).astype(np.float32)
    x = rng.standard_normal((5, cols)).astype(np.float32)
    m = fmat(w, s, rows, cols, br, bc)
    y = np.zeros((5, rows), np.float32)
    L.glm53f_mm_batch(y.ctypes.data, x.ctypes.data, 5, C.byref(m))
    assert same(y, O.mm_f8(O.oracle(), x, w, s, rows, cols, br, bc))
    y1 = np.zeros(rows, np.float32)
    L.glm53f_mm(y1.ctypes.data, np.ascontiguousarray(x[2]).ctypes.data, C.byref(m))
    assert same(y1, y[2])
    rows, cols = 96, 512
    q = rng.integers(0, 256, rows * cols // 2).astype(np.uint8)
    st = rng.uniform(1e-3, 1e-2, rows * cols // 64).astype(np.float32)
    xi = rng.standard_normal((5, cols)).astype(np.float32)
    mi = glm53h.Glm53fMat(q.ctypes.data, st.ctypes.data, glm53h.GLM53F_WI4, rows, cols, 1, 64, cols // 64)
    yi = np.zeros((5, rows), np.float32)
    L.glm53f_mm_batch(yi.ctypes.data, xi.ctypes.data, 5, C.byref(mi))
    assert same(yi, O.mm_i4(O.oracle(), xi, q, st, rows, cols))
