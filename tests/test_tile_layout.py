"""The octet-tiled code layout on the CPU (host twin of the conversion kernels): the conversion
round-trips, and every 16-byte run of a unit holds the codes one of the reference's eight fp32
accumulators of a 128-column block consumes, in the order it consumes them
(src/core/glm53f_ops.c:197-205: accumulator l takes columns l, l + 8, ..., l + 120)."""
import numpy as np

import glm53h


def tile(a, rows, cols, inverse=0):
    out = np.empty_like(a)
    assert glm53h.lib().g53h_tile_f8_host(out.ctypes.data, a.ctypes.data, rows, cols, inverse) == 0
    return out


def test_round_trip():
    rng = np.random.default_rng(1)
    for rows, cols in [(8, 128), (16, 256), (40, 640)]:
        a = rng.integers(0, 256, rows * cols, dtype=np.uint8)
        t = tile(a, rows, cols)
        assert not np.array_equal(t, a)
        assert np.array_equal(tile(t, rows, cols, 1), a)


def test_runs_are_accumulator_columns_in_order():
    rows, cols = 16, 256
    col = np.tile(np.arange(cols, dtype=np.int64), rows)
    row = np.repeat(np.arange(rows, dtype=np.int64), cols)
    for name, code in (("column", col % 256), ("row", row)):
        t = tile(code.astype(np.uint8), rows, cols)
        units = t.reshape(rows // 8, cols // 128, 8, 8, 16)      # octet, block, row, run, code
        for o8 in range(rows // 8):
            for b in range(cols // 128):
                for r in range(8):
                    accs = set()
                    for p in range(8):
                        run = units[o8, b, r, p].astype(np.int64)
                        if name == "row":
                            assert np.all(run == o8 * 8 + r)
                            continue
                        c = run - b * 128 if b * 128 < 256 else run
                        assert np.all(np.diff(c) == 8)             # consecutive columns of one accumulator
                        assert 0 <= c[0] < 8
                        accs.add(int(c[0]))
                        assert c[0] == glm53h_tile_acc(p)
                    if name == "column":
                        assert accs == set(range(8))


def glm53h_tile_acc(p):
    """The pairing of include/g53h.h: runs 0-3 accumulators 0 4 2 6, runs 4-7 1 5 3 7, so that
    the tree ((a0 + a4) + (a2 + a6)) + ((a1 + a5) + (a3 + a7)) pairs runs p and p ^ 1, then p and
    p ^ 2, then the two halves."""
    return [0, 4, 2, 6, 1, 5, 3, 7][p]


def test_tree_pairing():
    acc = [glm53h_tile_acc(p) for p in range(8)]
    level1 = {frozenset((acc[p], acc[p ^ 1])) for p in range(8)}
    assert level1 == {frozenset(s) for s in ((0, 4), (2, 6), (1, 5), (3, 7))}
    level2 = {frozenset(acc[q] for q in range(8) if q >> 2 == p >> 2) for p in range(8)}
    assert level2 == {frozenset((0, 4, 2, 6)), frozenset((1, 5, 3, 7))}


def mtile(a, rows, cols, inverse=0):
    out = np.empty_like(a)
    assert glm53h.lib().g53h_mtile_f8_host(out.ctypes.data, a.ctypes.data, rows, cols, inverse) == 0
    return out


def test_mfma_tiled_round_trip_and_operand_order():
    """MFMA-tiled units (G53H_MAT_MTILED): the same 1 KB unit grid as the octet-tiled layout, and
    lane 8 g + m of the unit's two 512-byte halves holds the 32 consecutive columns 32 g .. 32 g + 31
    of row m (16 in each half): the A operand of one 16 x 128 FP8 matrix-core tile."""
    rng = np.random.default_rng(2)
    for rows, cols in [(8, 128), (16, 256), (40, 640)]:
        a = rng.integers(0, 256, rows * cols, dtype=np.uint8)
        t = mtile(a, rows, cols)
        assert not np.array_equal(t, a)
        assert np.array_equal(mtile(t, rows, cols, 1), a)
    rows, cols = 16, 256
    r = np.repeat(np.arange(rows), cols)
    c = np.tile(np.arange(cols), rows)
    tr = mtile(r.astype(np.uint8), rows, cols).reshape(rows // 8, cols // 128, 2, 4, 8, 16)
    tc = mtile((c % 128).astype(np.uint8), rows, cols).reshape(rows // 8, cols // 128, 2, 4, 8, 16)
    tb = mtile((c // 128).astype(np.uint8), rows, cols).reshape(rows // 8, cols // 128, 2, 4, 8, 16)
    for o8 in range(rows // 8):
        for b in range(cols // 128):
            for g in range(4):
                for m in range(8):
                    lane_bytes = np.concatenate([tc[o8, b, 0, g, m], tc[o8, b, 1, g, m]])
                    assert np.array_equal(lane_bytes, np.arange(32 * g, 32 * g + 32))
                    assert np.all(tr[o8, b, :, g, m] == o8 * 8 + m)
                    assert np.all(tb[o8, b, :, g, m] == b)


def i4tile(a, rows, cols, inverse=0):
    out = np.zeros_like(a)
    assert glm53h.lib().g53h_tile_i4_host(out.ctypes.data, a.ctypes.data, rows, cols, inverse) == 0
    return out


def levels(packed, rows, cols):
    """Row-major int4 (the reference's GLM53F_WI4: low nibble = even column) to [rows][cols]."""
    b = packed.reshape(rows, cols // 2)
    out = np.empty((rows, cols), np.uint8)
    out[:, 0::2] = b & 15
    out[:, 1::2] = b >> 4
    return out


def test_int4_tiled_round_trip_and_accumulator_order():
    """Int4-tiled units (G53H_MAT_I4T): 8 rows x 256 columns per KB; run p of a unit row holds,
    for each of the block's four 64-column groups, the 8 levels of the reference's accumulator
    g53h_tile_acc(p) (columns acc + 8 i, i = 0..7, the order of matmul_i4's lane l,
    src/core/glm53f_ops.c:270-276), low nibble first."""
    rng = np.random.default_rng(4)
    for rows, cols in [(8, 256), (16, 512), (24, 768)]:
        a = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
        t = i4tile(a, rows, cols)
        assert not np.array_equal(t, a)
        assert np.array_equal(i4tile(t, rows, cols, 1), a)
        L = levels(a, rows, cols)
        w = t.view(np.uint32).reshape(rows // 8, cols // 256, 8, 8, 4)     # octet, block, row, run, group
        for o8 in range(rows // 8):
            for blk in range(cols // 256):
                for m in range(8):
                    for p in range(8):
                        acc = glm53h_tile_acc(p)
                        for g in range(4):
                            got = [(int(w[o8, blk, m, p, g]) >> (4 * i)) & 15 for i in range(8)]
                            want = L[o8 * 8 + m, blk * 256 + 64 * g + acc + 8 * np.arange(8)]
                            assert got == list(want)
    # every (row, group) holds the same 64 levels, so a group's dot product is unchanged
    rows, cols = 8, 256
    a = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    L = levels(a, rows, cols).astype(np.int64) - 8
    t = i4tile(a, rows, cols).view(np.uint32).reshape(8, 8, 4)
    x = rng.integers(-50, 50, cols)
    for m in range(8):
        for g in range(4):
            s = 0
            for p in range(8):
                acc = glm53h_tile_acc(p)
                for i in range(8):
                    s += (((int(t[m, p, g]) >> (4 * i)) & 15) - 8) * int(x[64 * g + acc + 8 * i])
            assert s == int(L[m, 64 * g:64 * g + 64] @ x[64 * g:64 * g + 64])


def test_int4_mfma_tiled_operand_order_and_steps():
    """Int4 MFMA-tiled units (G53H_MAT_I4 | G53H_MAT_MTILED): 8 rows x 128 columns per 512 bytes;
    lane slot 8 g + m holds row m's levels in the FP4 operand order of the matrix cores: nibble j
    (low first) is column 64 (g & 1) + 16 (g >> 1) + j for j < 16 and + 32 + (j - 16) after;
    the steps, 16 floats per unit, are [64-column half][row]."""
    lib = glm53h.lib()
    rng = np.random.default_rng(9)
    for rows, cols in [(8, 128), (16, 384), (24, 256)]:
        a = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
        st = rng.standard_normal(rows * (cols // 64)).astype(np.float32)
        t, ts = np.zeros_like(a), np.zeros_like(st)
        assert lib.g53h_mtile_i4_host(t.ctypes.data, ts.ctypes.data, a.ctypes.data, st.ctypes.data, rows, cols, 0) == 0
        back, bs = np.zeros_like(a), np.zeros_like(st)
        assert lib.g53h_mtile_i4_host(back.ctypes.data, bs.ctypes.data, t.ctypes.data, ts.ctypes.data, rows, cols, 1) == 0
        assert np.array_equal(back, a) and np.array_equal(bs, st)
        Lv = levels(a, rows, cols)
        S = st.reshape(rows, cols // 64)
        nb = cols // 128
        u8 = t.reshape(rows // 8, nb, 4, 8, 16)                     # octet, block, g, m, bytes
        us = ts.reshape(rows // 8, nb, 2, 8)                        # octet, block, half, row
        for o8 in range(rows // 8):
            for blk in range(nb):
                for g in range(4):
                    base = blk * 128 + 64 * (g & 1) + 16 * (g >> 1)
                    cols_j = [base + j if j < 16 else base + 32 + (j - 16) for j in range(32)]
                    for m in range(8):
                        by = u8[o8, blk, g, m]
                        nib = [(int(by[j // 2]) >> (4 * (j % 2))) & 15 for j in range(32)]
                        assert nib == list(Lv[o8 * 8 + m, cols_j])
                for hf in range(2):
                    assert np.array_equal(us[o8, blk, hf], S[o8 * 8:o8 * 8 + 8, 2 * blk + hf])
