"""The oracle's int4 expert path (or_i4_from_f8, or_mm_i4, or_moe_i4 in oracle/g53_oracle.c)
pinned before it is trusted: the reference's int4 known-answer inputs (tests/unit/test_fp8.c:
72-148, 158-161) against golden outputs of the compiled reference, the reference's own quantiser
property (every weight within half a step), a dequantise-then-fp64 bound, hand-made groups whose
levels and steps follow from the definition, and layer outputs of the compiled reference.
NaN codes are left out, as the reference's own quantiser test leaves them out
(tests/unit/test_fp8.c:118-121): its AVX2 and scalar builds treat them differently. No GPU."""
import ctypes as C
import hashlib
import os
import sys

import numpy as np
import pytest

import oracle_lib as O
import glm53h.synth as S

HERE = os.path.dirname(os.path.abspath(__file__))
G = np.load(os.path.join(HERE, "golden", "i4.npz"))
sys.path.insert(0, os.path.join(HERE, "golden"))
from make_i4 import NAL_CASES, nal_inputs  # noqa: E402


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def levels(q, cols):
    """Signed levels [rows][cols] of packed int4 rows."""
    q = np.asarray(q, np.uint8).reshape(-1, cols // 2)
    lv = np.empty((q.shape[0], cols), np.int64)
    lv[:, 0::2] = (q & 15).astype(np.int64) - 8
    lv[:, 1::2] = (q >> 4).astype(np.int64) - 8
    return lv


def dequant_f8(w, s, rows, cols, br, bc):
    from test_oracle import e4m3_closed_form
    tab = np.array([e4m3_closed_form(b) for b in range(256)])
    scols = (cols + bc - 1) // bc
    S2 = np.asarray(s, np.float64).reshape(-1, scols)
    r = np.arange(rows)[:, None] // br
    c = np.arange(cols)[None, :] // bc
    return tab[np.asarray(w).reshape(rows, cols)] * S2[r, c]


# ---------------------------------------------------------------- int4 matvec ----
def test_i4_matvec_known_answer_cases_bit_exact():
    cases, _ = O.i4_kat_cases()
    for i, c in enumerate(cases):
        y = O.mm_i4(O.oracle(), c["x"], c["q"], c["steps"], c["rows"], c["cols"])[0]
        assert np.array_equal(bits(y), bits(G[f"kat_i4_y{i}"])), (c["rows"], c["cols"])


def test_i4_matvec_against_fp64_dequantised_product():
    """y ~ sum_j (level_j * step_g) x_j in fp64: a swapped nibble, a wrong level offset or a wrong
    step index fails this at once."""
    rng = np.random.default_rng(5)
    rows, cols = 64, 1024
    q = rng.integers(0, 256, rows * cols // 2).astype(np.uint8)
    st = rng.uniform(1e-3, 1e-2, rows * cols // 64).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    y = O.mm_i4(O.oracle(), x, q, st, rows, cols)[0]
    W = levels(q, cols) * np.repeat(st.reshape(rows, -1).astype(np.float64), 64, axis=1)
    want = W @ x.astype(np.float64)
    assert np.allclose(y, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


def test_i4_matvec_batch_is_per_token():
    rng = np.random.default_rng(6)
    rows, cols = 32, 256
    q = rng.integers(0, 256, rows * cols // 2).astype(np.uint8)
    st = rng.uniform(1e-3, 1e-2, rows * cols // 64).astype(np.float32)
    x = rng.standard_normal((5, cols)).astype(np.float32)
    yb = O.mm_i4(O.oracle(), x, q, st, rows, cols)
    for t in range(5):
        assert np.array_equal(bits(yb[t]), bits(O.mm_i4(O.oracle(), x[t], q, st, rows, cols)[0]))


def test_i4_matvec_tail_of_ragged_group():
    """A group width that is not a multiple of 8 leaves a tail summed in double
    (src/core/glm53f_ops.c:283-287); the oracle with a 12-column group equals the closed form."""
    rng = np.random.default_rng(7)
    rows, cols, gs = 3, 24, 12
    q = rng.integers(0, 256, rows * cols // 2).astype(np.uint8)
    st = rng.uniform(0.5, 1.5, rows * (cols // gs)).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    y = np.empty(rows, np.float32)
    O.oracle().or_mm_i4(y.ctypes.data, x.ctypes.data, 1, q.ctypes.data, st.ctypes.data, rows, cols, gs)
    lv = levels(q, cols)
    for o in range(rows):
        acc = 0.0
        for g in range(cols // gs):
            a = np.zeros(8, np.float32)
            j0 = g * gs
            for l in range(8):
                a[l] = np.float32(np.float32(lv[o, j0 + l]) * x[j0 + l])    # one fused step from zero
            b = ((np.float64(a[0]) + a[4]) + (np.float64(a[2]) + a[6])) + ((np.float64(a[1]) + a[5]) +
                                                                           (np.float64(a[3]) + a[7]))
            for j in range(j0 + 8, j0 + gs):
                b += np.float64(lv[o, j]) * np.float64(x[j])
            acc += b * np.float64(st[o * (cols // gs) + g])
        assert bits(np.float32(acc)) == bits(y[o])


# ------------------------------------------------------------------ quantiser ----
def test_i4_quantiser_known_answer_case():
    _, c = O.i4_kat_cases()
    q, st = O.i4_from_f8(O.oracle(), c["w"], c["s"], c["rows"], c["cols"], c["br"], c["bc"])
    assert hashlib.sha256(q.tobytes()).digest() == G["kat_quant_q_sha"].tobytes()
    assert hashlib.sha256(st.tobytes()).digest() == G["kat_quant_steps_sha"].tobytes()
    assert np.array_equal(q[:8], G["kat_quant_q_head"])


def test_i4_quantiser_within_half_a_step():
    """The reference's own property (tests/unit/test_fp8.c:123-137): every weight within half a
    step of its FP8 value, with the levels in [-8, 7]."""
    _, c = O.i4_kat_cases()
    rows, cols = 64, c["cols"]
    w = c["w"][:rows * cols]
    q, st = O.i4_from_f8(O.oracle(), w, c["s"], rows, cols, c["br"], c["bc"])
    ref = dequant_f8(w, c["s"], rows, cols, c["br"], c["bc"])
    got = levels(q, cols) * np.repeat(st.astype(np.float64), 64, axis=1)
    step = np.repeat(st.astype(np.float64), 64, axis=1)
    assert np.all(np.abs(got - ref) <= 0.5 * step * 1.0001 + 1e-30)


def test_i4_quantiser_hand_made_groups():
    """Levels and steps that follow from the definition: the group maximum maps to +-7, an
    all-zero group gets the floor step 1e-30 and level 0 (byte 0x88), halves round to even."""
    cols = 128
    w = np.zeros((2, cols), np.uint8)
    # row 0, group 0: codes for +1.0 (0x38), -1.0 (0xb8) and 0.5 (0x30) -> levels 7, -7, rint(3.5) = 4
    w[0, 0], w[0, 1], w[0, 2] = 0x38, 0xb8, 0x30
    # row 0, group 1 left zero; row 1, group 0: 2.0 (0x40) and 1/7-step values
    w[1, 0], w[1, 3] = 0x40, 0x30          # 0.5 * 7 / 2 = 1.75 -> 2
    s = np.array([0.25], np.float32)        # one 128 x 128 block
    q, st = O.i4_from_f8(O.oracle(), w.ravel(), s, 2, cols, 128, 128)
    lv = levels(q, cols)
    assert lv[0, 0] == 7 and lv[0, 1] == -7 and lv[0, 2] == 4 and np.all(lv[0, 3:64] == 0)
    assert st[0, 0] == np.float32(np.float32(1.0 * 0.25) / np.float32(7.0))
    assert st[0, 1] == np.float32(1e-30) and np.all(q[0, 32:] == 0x88)
    assert lv[1, 0] == 7 and lv[1, 3] == 2
    assert st[1, 0] == np.float32(np.float32(2.0 * 0.25) / np.float32(7.0))


def test_i4_quantiser_unaligned_blocks_golden():
    for i, (rows, cols, br, bc, seed) in enumerate(NAL_CASES):
        w, s = nal_inputs(rows, cols, br, bc, seed)
        q, st = O.i4_from_f8(O.oracle(), w, s, rows, cols, br, bc)
        assert np.array_equal(q, G[f"nal{i}_q"]) and np.array_equal(bits(st), bits(G[f"nal{i}_steps"])), bc


@pytest.mark.skipif(not O.have_ref(), reason="reference not built")
def test_i4_quantiser_random_against_reference():
    rng = np.random.default_rng(9)
    for rows, cols, br, bc in [(24, 512, 8, 128), (5, 320, 2, 64), (7, 256, 3, 80)]:
        w = rng.integers(0, 256, rows * cols).astype(np.uint8)
        w[(w & 0x7f) == 0x7f] ^= 1
        s = rng.uniform(1e-5, 1e-1, ((rows + br - 1) // br) * ((cols + bc - 1) // bc)).astype(np.float32)
        a = O.i4_from_f8(O.oracle(), w, s, rows, cols, br, bc)
        b = O.i4_from_f8(O.ref(), w, s, rows, cols, br, bc)
        assert np.array_equal(a[0], b[0]) and np.array_equal(bits(a[1]), bits(b[1]))


# ---------------------------------------------------------------------- layer ----
def c1_i4():
    sp = S.spec(1)
    qm = {e: O.quantise_expert(O.oracle(), S.expert_host(sp, e), sp) for e in range(sp.NE)}
    return sp, S.router_host(sp), S.bias_host(sp), qm, S.expert_host(sp, "shared")


def test_moe_i4_config1_golden():
    sp, W, b, qm, sh = c1_i4()
    x = S.x_host(sp, 8, batch=0)
    out = np.stack([O.moe_i4(O.oracle(), x[t:t + 1], sp, W, b, qm, sh)[0][0] for t in range(8)])
    assert np.array_equal(bits(out), bits(G["c1_out"]))
    xb = S.x_host(sp, 5, batch=1)
    assert np.array_equal(bits(O.moe_i4(O.oracle(), xb, sp, W, b, qm, sh)[0]), bits(G["c1b_out"]))
    assert np.array_equal(bits(O.moe_i4(O.oracle(), xb, sp, W, b, qm, None)[0]), bits(G["c1b_routed_out"]))


def test_moe_i4_config2_one_token_golden():
    sp = S.spec(2)
    W, b = S.router_host(sp), S.bias_host(sp)
    x = S.x_host(sp, 1, batch=0)
    idx, _ = O.router(O.oracle(), x, sp, W, b)
    qm = {int(e): O.quantise_expert(O.oracle(), S.expert_host(sp, int(e)), sp) for e in idx[0]}
    out = O.moe_i4(O.oracle(), x, sp, W, b, qm, S.expert_host(sp, "shared"))[0][0]
    assert np.array_equal(bits(out), bits(G["c2_out"]))


def test_moe_i4_is_weighted_sum_of_int4_experts():
    """The int4 layer equals sum_j w_j expert_j(x) over int4 experts run on their own, plus the
    FP8 shared expert (an FP8 routed product or a dropped shared term fails)."""
    from test_oracle import run_expert
    sp, W, b, qm, sh = c1_i4()
    x = S.x_host(sp, 1, batch=3)
    out, idx, w = O.moe_i4(O.oracle(), x, sp, W, b, qm, sh)
    acc = np.zeros(sp.E)
    for j, e in enumerate(idx[0]):
        (gq, gs), (uq, us), (dq, ds) = qm[int(e)]
        g = O.mm_i4(O.oracle(), x, gq, gs, sp.I, sp.E)[0]
        u = O.mm_i4(O.oracle(), x, uq, us, sp.I, sp.E)[0]
        a = np.empty(sp.I, np.float32)
        gu = np.concatenate([g, u])
        O.oracle().or_swiglu(a.ctypes.data, gu.ctypes.data, sp.I, C.c_float(sp.limit))
        acc += np.float64(w[0][j]) * O.mm_i4(O.oracle(), a, dq, ds, sp.E, sp.I)[0]
    acc += run_expert(sp, x, sh)
    assert np.allclose(out[0], acc, rtol=1e-5, atol=1e-7)
