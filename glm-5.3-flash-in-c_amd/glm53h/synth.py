"""Seeded synthetic MoE layers on the host and in HBM.

Every array is a pure function of (seed, stream); the streams below fix which stream each
tensor draws from, so tests, golden fixtures, the bench and the CPU baseline all see the same
inputs. Large expert weights are generated in HBM by the device generator; the host twin
(g53h_synth_f8_host) yields the same bytes for the few experts a CPU check needs.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field

import numpy as np

from . import G53hExpert, G53hMat, G53hMoeLayer, DevBuf, check, lib

K_ROUTER, K_BIAS, K_X, K_EXPERT, K_SHARED = 1, 2, 3, 4, 5


def stream(kind, layer=0, index=0):
    return (layer << 40) | (kind << 32) | index


@dataclass
class LayerSpec:
    E: int = 256
    I: int = 128
    NE: int = 16
    K: int = 8
    norm_topk: int = 1
    routed_scale: float = 2.5
    limit: float = 10.0
    br: int = 128
    bc: int = 128
    router_sigma: float = 0.02
    expert_sigma: float = 0.02
    bias_a: float = 0.1
    zipf_s: float | None = None      # Zipf exponent of the popularity skew, None = uniform
    seed: int = 1
    layer: int = 0
    shared: bool = True

    def expert_bytes(self):
        """Codes + scales of one expert (BASELINE's 25,171,968 B at the released shapes)."""
        sr = lambda r, c: ((r + self.br - 1) // self.br) * ((c + self.bc - 1) // self.bc) * 4
        return 3 * self.E * self.I + 2 * sr(self.I, self.E) + sr(self.E, self.I)

    def expert_i4_bytes(self):
        """Levels + steps of one int4 expert (14,155,776 B at the released shapes)."""
        return 3 * (self.E * self.I // 2) + 3 * (self.E * self.I // 64) * 4


CONFIG1 = dict(E=256, I=128, NE=16, K=8, router_sigma=0.02)
CONFIG2 = dict(E=4096, I=2048, NE=288, K=8, router_sigma=1.0 / 64.0)


def spec(config, **kw):
    base = {1: CONFIG1, 2: CONFIG2, 3: CONFIG2, 4: CONFIG2, 5: CONFIG2}[config]
    d = dict(base)
    if config == 3:
        d["zipf_s"] = 1.1
    d.update(kw)
    return LayerSpec(**d)


# ------------------------------------------------------------------------ host ----
def normal_host(n, seed, strm, sigma, bf16):
    out = np.empty(n, np.float32)
    lib().g53h_synth_normal_host(out.ctypes.data, n, seed, strm, C.c_float(sigma), int(bf16))
    return out


def router_host(sp: LayerSpec):
    """Router [NE][E] fp32 holding bf16 values (the checkpoint's router is bf16)."""
    return normal_host(sp.NE * sp.E, sp.seed, stream(K_ROUTER, sp.layer), sp.router_sigma, True).reshape(sp.NE, sp.E)


def bias_host(sp: LayerSpec):
    """Selection bias [NE]: U(-a, a), or for a Zipf(s) popularity the calibrated bias-by-rank
    curve of glm53h.zipf (top-k selection probability min(1, c rank^-s)) over a seeded
    permutation of ranks, one permutation per layer."""
    if sp.zipf_s is None:
        out = np.empty(sp.NE, np.float32)
        lib().g53h_synth_uniform_host(out.ctypes.data, sp.NE, sp.seed, stream(K_BIAS, sp.layer),
                                      C.c_float(sp.bias_a))
        return out
    from . import zipf
    curve = np.asarray(zipf.table(sp.NE, sp.K, sp.zipf_s)["bias_by_rank"], np.float64)
    rng = np.random.default_rng(sp.seed * 1000003 + sp.layer)
    rank = rng.permutation(sp.NE)                  # expert e has popularity rank rank[e] + 1
    return curve[rank].astype(np.float32)


def x_host(sp: LayerSpec, T, batch=0):
    """Activations [T][E], bf16 values N(0, 1), as fp32."""
    return normal_host(T * sp.E, sp.seed, stream(K_X, sp.layer, batch), 1.0, True).reshape(T, sp.E)


def _mat_shapes(sp):
    return [(sp.I, sp.E), (sp.I, sp.E), (sp.E, sp.I)]


def expert_host(sp: LayerSpec, e):
    """Expert e (or the shared expert for e == 'shared') as [(codes, scales)] x 3 on the host."""
    mats = []
    for m, (r, c) in enumerate(_mat_shapes(sp)):
        strm = stream(K_SHARED, sp.layer, m) if e == "shared" else stream(K_EXPERT, sp.layer, e * 3 + m)
        w = np.empty(r * c, np.uint8)
        s = np.empty(((r + sp.br - 1) // sp.br) * ((c + sp.bc - 1) // sp.bc), np.float32)
        lib().g53h_synth_f8_host(w.ctypes.data, s.ctypes.data, r, c, sp.br, sp.bc, sp.seed, strm,
                                 C.c_float(sp.expert_sigma))
        mats.append((w, s))
    return mats


# ---------------------------------------------------------------------- device ----
def _align(v, a=256):
    return (v + a - 1) // a * a


@dataclass
class DeviceLayer:
    """One MoE layer resident in HBM: router (bf16), bias, every expert in a slot of one arena
    (codes of gate, up, down, then their scales, as the reference's expert slot), the shared
    expert, and the device table of expert descriptors."""
    sp: LayerSpec
    arena: DevBuf = None
    slot_bytes: int = 0
    router: DevBuf = None
    bias: DevBuf = None
    table: DevBuf = None
    experts: list = field(default_factory=list)
    layer: G53hMoeLayer = None
    router_f32: np.ndarray = None
    bias_f32: np.ndarray = None

    tiled: bool = False
    i4: bool = False
    mfma: bool = False
    i4t: bool = False

    @classmethod
    def build(cls, sp: LayerSpec, n_experts_present=None, tiled=False, i4=False, mfma=False):
        """tiled: store every expert's codes octet-tiled (G53H_MAT_TILED), the layout the decode
        kernel k_dec_tiled streams; the values are the same seeded codes either way.
        mfma: MFMA-tiled instead (G53H_MAT_MTILED), the layout of k_dec_mfma.
        i4: re-quantise every routed expert on the device into the reference's int4 format
        (G53H_MAT_I4: levels, and one step per row and 64 columns; the reference's
        --experts int4), the shared expert staying FP8; the layer then has block_c 0.
        i4 and tiled: the int4 levels int4-tiled (G53H_MAT_I4T), the layout of the one-launch
        int4 decode, and the shared expert octet-tiled; the layer has tiled 3, block_c 128.
        i4 and mfma: the int4 levels and steps int4 MFMA-tiled (G53H_MAT_I4 | G53H_MAT_MTILED), the
        layout of the FP4 matrix-core decode, and the shared expert FP8 MFMA-tiled; tiled 4."""
        assert not (mfma and tiled)
        self = cls(sp)
        self.i4m = bool(mfma and i4)
        self.i4t = bool(tiled and i4)
        if self.i4t:
            tiled = False
        self.mfma = bool(mfma)
        tiled = tiled or mfma
        self.tiled = bool(tiled)
        self.i4 = bool(i4)
        E, I, NE = sp.E, sp.I, sp.NE
        shapes = _mat_shapes(sp)
        code_off, sc_off, off = [], [], 0
        for r, c in shapes:
            code_off.append(off)
            off = _align(off + r * c)
        for r, c in shapes:
            sc_off.append(off)
            off = _align(off + ((r + sp.br - 1) // sp.br) * ((c + sp.bc - 1) // sp.bc) * 4)
        self.slot_bytes = _align(off, 4096)
        nslots = NE + (1 if sp.shared else 0)
        self.arena = DevBuf(self.slot_bytes * nslots)
        L = lib()
        descs = (G53hExpert * (NE + 1))()
        stage = DevBuf(max(r * c for r, c in shapes)) if self.tiled else None
        if self.i4:                              # FP8 staging of one matrix and its scales
            s_stage = _align(max(r * c for r, c in shapes))
            stage = DevBuf(s_stage + max(((r + sp.br - 1) // sp.br) * ((c + sp.bc - 1) // sp.bc) * 4
                                         for r, c in shapes))
            stage4 = DevBuf(max(r * c // 2 for r, c in shapes)) if (self.i4t or self.i4m) else None
            stage4s = DevBuf(max(r * (c // 64) * 4 for r, c in shapes)) if self.i4m else None
        for i in range(nslots):
            base = self.arena.ptr + i * self.slot_bytes
            mats = []
            if self.i4 and i < NE:
                off4 = 0
                for m, (r, c) in enumerate(shapes):
                    strm = stream(K_EXPERT, sp.layer, i * 3 + m)
                    check(L.g53h_synth_f8(stage.ptr, stage.ptr + s_stage, r, c, sp.br, sp.bc, sp.seed, strm,
                                          C.c_float(sp.expert_sigma)), "g53h_synth_f8")
                    f = G53hMat(stage.ptr, stage.ptr + s_stage, r, c, sp.br, sp.bc, (c + sp.bc - 1) // sp.bc, 0)
                    q = base + off4
                    off4 = _align(off4 + r * c // 2)
                    st = base + off4
                    off4 = _align(off4 + r * (c // 64) * 4)
                    if self.i4t:                 # quantised row-major into staging, then tiled
                        check(L.g53h_i4_from_f8(stage4.ptr, st, C.byref(f)), "g53h_i4_from_f8")
                        check(L.g53h_tile_i4(q, stage4.ptr, r, c, 0), "g53h_tile_i4")
                    elif self.i4m:               # levels and steps into staging, then MFMA-tiled
                        check(L.g53h_i4_from_f8(stage4.ptr, stage4s.ptr, C.byref(f)), "g53h_i4_from_f8")
                        check(L.g53h_mtile_i4(q, st, stage4.ptr, stage4s.ptr, r, c, 0), "g53h_mtile_i4")
                    else:
                        check(L.g53h_i4_from_f8(q, st, C.byref(f)), "g53h_i4_from_f8")
                    mats.append(G53hMat(q, st, r, c, 1, 64, c // 64,
                                        4 | (16 if self.i4t else 0) | (8 if self.i4m else 0)))
                descs[i] = G53hExpert(*mats)
                continue
            # an int4 layer keeps its FP8 shared expert octet-tiled where the shapes allow (the
            # row-wave kernel's fast FP8 path), as the drop-in does
            tile = self.tiled or (self.i4 and sp.bc == 128 and all(r % 8 == 0 and c % 128 == 0 for r, c in shapes))
            assert tile or not (self.i4t or self.i4m), "the int4-tiled layer needs a tiled shared expert"
            for m, (r, c) in enumerate(shapes):
                strm = stream(K_SHARED, sp.layer, m) if i == NE else stream(K_EXPERT, sp.layer, i * 3 + m)
                w, s = base + code_off[m], base + sc_off[m]
                gen = stage.ptr if tile else w
                check(L.g53h_synth_f8(gen, s, r, c, sp.br, sp.bc, sp.seed, strm, C.c_float(sp.expert_sigma)),
                      "g53h_synth_f8")
                if tile and self.mfma:
                    check(L.g53h_mtile_f8(w, gen, r, c, 0), "g53h_mtile_f8")
                elif tile:
                    check(L.g53h_tile_f8(w, gen, r, c), "g53h_tile_f8")
                flag = (8 if self.mfma else 2) if tile else 0
                mats.append(G53hMat(w, s, r, c, sp.br, sp.bc, (c + sp.bc - 1) // sp.bc, flag))
            descs[i] = G53hExpert(*mats)
        self.experts = descs
        self.table = DevBuf.from_array(np.frombuffer(bytes(descs), np.uint8))
        self.router_f32 = router_host(sp)
        rb = (self.router_f32.view(np.uint32) >> 16).astype(np.uint16)
        self.router = DevBuf.from_array(rb)
        self.bias_f32 = bias_host(sp)
        self.bias = DevBuf.from_array(self.bias_f32)
        self.layer = G53hMoeLayer(
            hidden=E, inter=I, n_experts=NE, topk=sp.K, norm_topk=sp.norm_topk,
            routed_scale=sp.routed_scale, swiglu_limit=sp.limit, router=self.router.ptr, router_dt=1,
            bias=self.bias.ptr, experts=self.table.ptr,
            shared=(self.table.ptr + NE * C.sizeof(G53hExpert)) if sp.shared else None,
            block_c=sp.bc if (self.i4t or self.i4m) else (0 if self.i4 else sp.bc),
            tiled=4 if self.i4m else (3 if self.i4t else ((2 if self.mfma else 1) if self.tiled else 0)))
        check(L.g53h_sync(), "g53h_sync")
        del stage
        return self

    def fetch_expert(self, e):
        """[(codes, scales)] x 3 of expert e (or 'shared') copied back from HBM."""
        d = self.experts[self.sp.NE if e == "shared" else e]
        out = []
        for m in (d.gate, d.up, d.down):
            if m.flags & 4:                       # int4: levels [rows][cols/2], steps [rows][scols]
                w = np.empty(m.rows * (m.cols // 2), np.uint8)
                s = np.empty(m.rows * m.scols, np.float32)
                check(lib().g53h_d2h(w.ctypes.data, m.w, w.nbytes), "d2h")
                check(lib().g53h_d2h(s.ctypes.data, m.s, s.nbytes), "d2h")
                if m.flags & 16:                  # int4-tiled in HBM: the row-major levels
                    rm = np.zeros_like(w)
                    assert lib().g53h_tile_i4_host(rm.ctypes.data, w.ctypes.data, m.rows, m.cols, 1) == 0
                    w = rm
                elif m.flags & 8:                 # int4 MFMA-tiled: levels and steps row-major
                    rm, rs = np.zeros_like(w), np.zeros_like(s)
                    assert lib().g53h_mtile_i4_host(rm.ctypes.data, rs.ctypes.data, w.ctypes.data, s.ctypes.data,
                                                    m.rows, m.cols, 1) == 0
                    w, s = rm, rs
                out.append((w, s))
                continue
            w = np.empty(m.rows * m.cols, np.uint8)
            s = np.empty(((m.rows + m.br - 1) // m.br) * m.scols, np.float32)
            check(lib().g53h_d2h(w.ctypes.data, m.w, w.nbytes), "d2h")
            check(lib().g53h_d2h(s.ctypes.data, m.s, s.nbytes), "d2h")
            if m.flags & 2:                       # tiled in HBM: the row-major codes for the oracle
                rm = np.empty_like(w)
                assert lib().g53h_tile_f8_host(rm.ctypes.data, w.ctypes.data, m.rows, m.cols, 1) == 0
                w = rm
            elif m.flags & 8:                     # MFMA-tiled
                rm = np.empty_like(w)
                assert lib().g53h_mtile_f8_host(rm.ctypes.data, w.ctypes.data, m.rows, m.cols, 1) == 0
                w = rm
            out.append((w, s))
        return out

    def forward(self, out: DevBuf, x: DevBuf, T, idx: DevBuf = None, w: DevBuf = None):
        check(lib().g53h_moe(out.ptr, x.ptr, T, C.byref(self.layer), idx.ptr if idx else None,
                             w.ptr if w else None), "g53h_moe")

    def algorithmic_bytes(self, n_unique_routed):
        """HBM bytes one layer call must read: each unique routed expert and the shared expert
        once, the bf16 router and the bias."""
        sp = self.sp
        routed = sp.expert_i4_bytes() if self.i4 else sp.expert_bytes()
        return n_unique_routed * routed + (sp.expert_bytes() if sp.shared else 0) + sp.NE * sp.E * 2 + sp.NE * 4
