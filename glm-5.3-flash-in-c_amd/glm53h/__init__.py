"""glm53h - Python host binding of the MI355X routed-expert MoE library (lib/libglm53h.so).

The product is the C-ABI shared library: gfx950 HIP kernels behind include/g53h.h, and the
reference engine's expert-path entry points (include/glm53f.h) written in C over it. This
module loads that library with ctypes and mirrors its structs so that tests and the bench can
drive it; it performs no arithmetic of its own. There is no fallback: if the library is not
built, or no GPU is present when a device call is made, it raises.

PyTorch is deliberately not imported in a process that loads this library: PyTorch ships its
own HIP runtime, and two HIP runtimes in one process do not share devices or pointers.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("G53H_LIB") or os.path.join(PKG_DIR, "lib", "libglm53h.so")
INCLUDE_DIR = os.path.join(os.path.dirname(PKG_DIR), "include")

_lib = None


class G53hError(RuntimeError):
    pass


# ----------------------------------------------------------------- structs (g53h.h) ----
class G53hMat(C.Structure):
    _fields_ = [("w", C.c_void_p), ("s", C.c_void_p), ("rows", C.c_int), ("cols", C.c_int),
                ("br", C.c_int), ("bc", C.c_int), ("scols", C.c_int), ("flags", C.c_int)]


class G53hExpert(C.Structure):
    _fields_ = [("gate", G53hMat), ("up", G53hMat), ("down", G53hMat)]


class G53hMoeLayer(C.Structure):
    _fields_ = [("hidden", C.c_int), ("inter", C.c_int), ("n_experts", C.c_int),
                ("topk", C.c_int), ("norm_topk", C.c_int), ("routed_scale", C.c_float),
                ("swiglu_limit", C.c_float), ("router", C.c_void_p), ("router_dt", C.c_int),
                ("bias", C.c_void_p), ("experts", C.c_void_p), ("shared", C.c_void_p),
                ("block_c", C.c_int), ("tiled", C.c_int)]


# -------------------------------------------------------------- structs (glm53f.h) ----
GLM53F_MAX_LAYERS = 256
GLM53F_MAX_EOS = 8
GLM53F_WF32, GLM53F_WBF16, GLM53F_WF8, GLM53F_WI4, GLM53F_WF8T, GLM53F_WI4T, GLM53F_WI4M, GLM53F_WF8M = (
    0, 1, 2, 3, 0x102, 0x103, 0x104, 0x105)


class Glm53fCfg(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("hidden", "n_layers", "vocab")] + [
        ("rms_eps", C.c_float), ("hc_mult", C.c_int), ("hc_iters", C.c_int), ("hc_eps", C.c_float),
        ("kda_heads", C.c_int), ("kda_head_dim", C.c_int), ("conv_k", C.c_int),
        ("gate_lb", C.c_float)] + [(n, C.c_int) for n in (
            "n_heads", "q_lora", "kv_lora", "qk_nope", "v_head", "index_topk", "index_kpool",
            "index_heads", "index_dim", "index_tail", "n_experts", "topk", "n_shared",
            "moe_inter", "dense_inter")] + [
        ("routed_scale", C.c_float), ("norm_topk", C.c_int), ("swiglu_limit", C.c_float),
        ("fp8_block_r", C.c_int), ("fp8_block_c", C.c_int),
        ("is_mla", C.c_ubyte * GLM53F_MAX_LAYERS), ("is_dense", C.c_ubyte * GLM53F_MAX_LAYERS),
        ("eos", C.c_int * GLM53F_MAX_EOS), ("n_eos", C.c_int)]


class Glm53fMat(C.Structure):
    _fields_ = [("w", C.c_void_p), ("s", C.c_void_p), ("dt", C.c_int), ("rows", C.c_int),
                ("cols", C.c_int), ("br", C.c_int), ("bc", C.c_int), ("scols", C.c_int)]


class Glm53fExpertQ(C.Structure):
    _fields_ = [("gate", Glm53fMat), ("up", Glm53fMat), ("down", Glm53fMat)]


class Glm53fExpertSrc(C.Structure):
    pass


GET_FN = C.CFUNCTYPE(C.c_int, C.POINTER(Glm53fExpertSrc), C.c_int, C.c_int, C.POINTER(Glm53fExpertQ))
GETMANY_FN = C.CFUNCTYPE(C.c_int, C.POINTER(Glm53fExpertSrc), C.c_int, C.POINTER(C.c_int), C.c_int)
RELEASE_FN = C.CFUNCTYPE(None, C.POINTER(Glm53fExpertSrc), C.c_int, C.c_int)
HINT_FN = C.CFUNCTYPE(None, C.POINTER(Glm53fExpertSrc), C.c_int, C.POINTER(C.c_int), C.c_int)

Glm53fExpertSrc._fields_ = [("get", GET_FN), ("getmany", GETMANY_FN), ("release", RELEASE_FN),
                            ("hint", HINT_FN), ("ctx", C.c_void_p)]


class Glm53fMoeW(C.Structure):
    _fields_ = [("gate", C.c_void_p), ("bias", C.c_void_p), ("sh_gate", Glm53fMat),
                ("sh_up", Glm53fMat), ("sh_down", Glm53fMat),
                ("src", C.POINTER(Glm53fExpertSrc)), ("next_gate", C.c_void_p),
                ("next_bias", C.c_void_p), ("ahead_gate", C.c_void_p * 3),
                ("ahead_bias", C.c_void_p * 3), ("prefetch_n", C.c_int),
                ("prefill_next", C.c_int), ("layer", C.c_int)]


VIEW_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.c_int, C.POINTER(Glm53fExpertQ))
DONE_FN = C.CFUNCTYPE(None, C.c_void_p, C.c_int, C.c_int)


class G53hStore(C.Structure):
    """include/glm53f_cache.h: a source of host-resident experts for g53h_cache_init_store."""
    _fields_ = [("view", VIEW_FN), ("done", DONE_FN), ("ctx", C.c_void_p)]


class Glm53fTensor(C.Structure):
    """include/glm53f_st.h (the reference reader's Glm53fTensor)."""
    _fields_ = [("name", C.c_char_p), ("shard", C.c_int), ("dtype", C.c_int), ("ndim", C.c_int),
                ("shape", C.c_int64 * 8), ("off", C.c_int64), ("nbytes", C.c_int64)]


class Glm53fSt(C.Structure):
    """include/glm53f_st.h (the reference reader's Glm53fSt): the checkpoint index."""
    _fields_ = [("fd", C.POINTER(C.c_int)), ("dfd", C.POINTER(C.c_int)), ("path", C.POINTER(C.c_char_p)),
                ("nshard", C.c_int), ("t", C.POINTER(Glm53fTensor)), ("nt", C.c_int),
                ("bucket", C.POINTER(C.c_int32)), ("nbucket", C.c_int), ("strpool", C.c_void_p),
                ("strcap", C.c_size_t), ("strlen_", C.c_size_t)]


_COND, _MUTEX = C.c_int64 * 6, C.c_int64 * 5        # glibc x86-64 pthread_cond_t, pthread_mutex_t (8-aligned)


class Glm53fCache(C.Structure):
    """include/glm53f_cache.h: the reference's Glm53fCache layout (src must stay first)."""
    _fields_ = [("src", Glm53fExpertSrc), ("st", C.c_void_p), ("cfg", C.c_void_p),
                ("n_layers", C.c_int), ("n_experts", C.c_int), ("arena", C.c_void_p), ("slot_bytes", C.c_int64),
                ("nslot", C.c_int), ("i4", C.c_int), ("raw_bytes", C.c_int64), ("stage", C.c_void_p),
                ("stage_busy", C.c_void_p), ("nstage", C.c_int), ("stage_free", _COND), ("i4_fd", C.c_void_p),
                ("i4_layers", C.c_int), ("slot_of", C.POINTER(C.c_int32)), ("inflight_of", C.POINTER(C.c_int32)),
                ("key_of", C.POINTER(C.c_int32)), ("pins", C.POINTER(C.c_int32)), ("prefetched", C.c_void_p),
                ("used_at", C.POINTER(C.c_uint64)), ("ref", C.c_void_p), ("pad", C.c_void_p),
                ("clock", C.c_uint64), ("mu", _MUTEX), ("landed", _COND), ("work", _COND), ("n_io", C.c_int),
                ("io", C.c_void_p), ("stop", C.c_int), ("queue", C.c_void_p), ("qcap", C.c_int), ("qlen", C.c_int),
                ("hint_floor", C.c_int), ("last_hint", C.c_int), ("queued", C.c_void_p),
                ("hits", C.c_uint64), ("misses", C.c_uint64), ("evictions", C.c_uint64),
                ("bytes_read", C.c_uint64), ("prefetch_reads", C.c_uint64), ("load_seconds", C.c_double),
                ("bg_reads", C.c_uint64), ("bg_bytes", C.c_uint64), ("bg_used", C.c_uint64)]


# ------------------------------------------------------------------- loading ----
_SIGS = {
    # runtime
    "g53h_init": (C.c_int, [C.c_int]),
    "g53h_device_count": (C.c_int, []),
    "g53h_error": (C.c_char_p, []),
    "g53h_sync": (C.c_int, []),
    "g53h_alloc": (C.c_void_p, [C.c_size_t]),
    "g53h_free": (C.c_int, [C.c_void_p]),
    "g53h_host_alloc": (C.c_void_p, [C.c_size_t]),
    "g53h_host_free": (C.c_int, [C.c_void_p]),
    "g53h_h2d": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "g53h_d2h": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "g53h_d2d": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "g53h_h2d_async": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "g53h_memset": (C.c_int, [C.c_void_p, C.c_int, C.c_size_t]),
    "g53h_is_device_ptr": (C.c_int, [C.c_void_p]),
    "g53h_mark": (C.c_int, []),
    "g53h_elapsed_ms": (C.c_float, []),
    "g53h_prof_enable": (C.c_int, [C.c_int]),
    "g53h_prof_collect": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int]),
    "g53h_mem_info": (C.c_int, [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    # ops
    "g53h_mm_f8": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.POINTER(G53hMat)]),
    "g53h_i4_from_f8": (C.c_int, [C.c_void_p, C.c_void_p, C.POINTER(G53hMat)]),
    "g53h_swiglu": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_float]),
    "g53h_router": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int,
                              C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_void_p]),
    "g53h_route_decode": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p,
                                    C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                    C.c_int, C.c_float, C.c_int, C.c_uint, C.c_size_t]),
    "g53h_route_topn": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                                  C.c_int, C.c_int]),
    "g53h_moe": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.POINTER(G53hMoeLayer), C.c_void_p,
                           C.c_void_p]),
    "g53h_moe_routed_given": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.POINTER(G53hMoeLayer),
                                        C.c_void_p, C.c_void_p]),
    "g53h_moe_partial": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.POINTER(G53hMoeLayer),
                                   C.c_void_p]),
    "g53h_moe_combine": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                                   C.POINTER(G53hMoeLayer)]),
    "g53h_moe_grouped": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.POINTER(G53hMoeLayer), C.c_void_p,
                                   C.c_void_p]),
    "g53h_set_grouped": (C.c_int, [C.c_int]),
    "g53h_grouped_max_tokens": (C.c_int, [C.POINTER(G53hMoeLayer)]),
    "g53h_grouped_begin": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(G53hMoeLayer), C.c_void_p]),
    "g53h_grouped_batch": (C.c_int, [C.POINTER(G53hMoeLayer)]),
    "g53h_grouped_end": (C.c_int, [C.c_void_p, C.c_void_p]),
    "g53h_grouped_ok": (C.c_int, [C.POINTER(G53hMoeLayer)]),
    "g53h_grouped_errors": (C.c_int, []),
    "g53h_set_grouped_trace": (C.c_int, [C.c_void_p]),
    "g53h_set_fused_decode": (C.c_int, [C.c_int]),
    "g53h_decode_errors": (C.c_int, []),
    "g53h_decode_grid": (C.c_int, []),
    "g53h_set_decode_trace": (C.c_int, [C.c_void_p]),
    "g53h_errors_async": (C.c_int, [C.c_void_p]),
    "g53h_route_topn_batch": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int,
                                        C.c_void_p, C.c_int, C.c_int]),
    "g53h_vote": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    "g53h_set_spin_limit": (C.c_int, [C.c_int]),
    "g53h_inject_errors": (C.c_int, [C.c_int, C.c_int]),
    "g53h_errors_peek_async": (C.c_int, [C.c_void_p]),
    "g53h_mailbox": (C.c_void_p, []),
    "g53h_mailbox_wait": (C.c_int, [C.c_int, C.c_uint]),
    "g53h_publish": (C.c_int, [C.c_int, C.c_uint, C.c_size_t, C.c_void_p, C.c_size_t]),
    "g53h_inbox": (C.c_void_p, []),
    "g53h_inbox_fetch": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t]),
    "g53h_route_next": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int]),
    "g53h_decode_next": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int]),
    "g53h_decode_publish": (C.c_int, [C.c_int, C.c_uint, C.c_size_t, C.c_void_p, C.c_int, C.c_void_p, C.c_int,
                                      C.c_int, C.c_size_t, C.c_void_p, C.c_size_t]),
    "g53h_d2h_async": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "g53h_moe_decode_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.POINTER(G53hMoeLayer), C.c_void_p, C.c_void_p]),
    "g53h_set_tiled_decode_trace": (C.c_int, [C.c_void_p]),
    "g53h_set_mfma_decode_trace": (C.c_int, [C.c_void_p]),
    "g53h_mtile_f8": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    "g53h_mtile_f8_host": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    "g53h_tile_i4": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    "g53h_tile_i4_host": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    "g53h_mtile_i4": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    "g53h_mtile_i4_host": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    "g53h_tile_f8": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int]),
    "g53h_untile_f8": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int]),
    "g53h_tile_f8_host": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    "g53h_expf": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "g53h_expf_range": (C.c_int, [C.c_void_p, C.c_uint32, C.c_size_t]),
    "g53h_expf_host": (None, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "g53h_e4m3_decode": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "g53h_synth_f8": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int,
                                C.c_uint64, C.c_uint64, C.c_float]),
    "g53h_synth_f8_host": (None, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int,
                                  C.c_uint64, C.c_uint64, C.c_float]),
    "g53h_synth_normal_host": (None, [C.c_void_p, C.c_size_t, C.c_uint64, C.c_uint64, C.c_float,
                                      C.c_int]),
    "g53h_quant_host": (None, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_float]),
    "g53h_synth_uniform_host": (None, [C.c_void_p, C.c_size_t, C.c_uint64, C.c_uint64, C.c_float]),
    # drop-in (glm53f.h)
    "glm53f_mm": (None, [C.c_void_p, C.c_void_p, C.POINTER(Glm53fMat)]),
    "glm53f_i4_from_f8": (None, [C.c_void_p, C.c_void_p, C.POINTER(Glm53fMat)]),
    "glm53f_mm_batch": (None, [C.c_void_p, C.c_void_p, C.c_int, C.POINTER(Glm53fMat)]),
    "glm53f_e4m3f": (C.c_float, [C.c_uint8]),
    "glm53f_swiglu_clamp": (None, [C.c_void_p, C.c_void_p, C.c_int, C.c_float]),
    "glm53f_router": (None, [C.c_void_p, C.c_void_p, C.c_void_p, C.POINTER(Glm53fMoeW),
                             C.POINTER(Glm53fCfg)]),
    "glm53f_moe_scratch": (C.c_size_t, [C.POINTER(Glm53fCfg), C.c_int]),
    "glm53f_moe": (None, [C.c_void_p, C.c_void_p, C.POINTER(Glm53fMoeW), C.POINTER(Glm53fCfg),
                          C.c_int, C.c_void_p]),
    "glm53f_moe_routed": (None, [C.c_void_p, C.c_void_p, C.POINTER(Glm53fMoeW),
                                 C.POINTER(Glm53fCfg), C.c_int, C.c_void_p]),
    "glm53f_mlp_scratch": (C.c_size_t, [C.POINTER(Glm53fCfg)]),
    "glm53f_mlp": (None, [C.c_void_p, C.c_void_p, C.POINTER(Glm53fMat), C.POINTER(Glm53fMat),
                          C.POINTER(Glm53fMat), C.c_float, C.c_void_p]),
    "glm53f_forget_host_weights": (None, []),
    # expert cache (glm53f_cache.h)
    "glm53f_cache_init": (C.c_int, [C.POINTER(Glm53fCache), C.POINTER(Glm53fSt), C.POINTER(Glm53fCfg), C.c_int64,
                                    C.c_int, C.c_int]),
    "glm53f_cache_free": (None, [C.POINTER(Glm53fCache)]),
    "glm53f_cache_reset_stats": (None, [C.POINTER(Glm53fCache)]),
    "glm53f_cache_report": (None, [C.POINTER(Glm53fCache), C.c_char_p]),
    "glm53f_cache_sync": (C.c_int, [C.POINTER(Glm53fCache)]),
    "g53h_cache_is": (C.c_int, [C.POINTER(Glm53fExpertSrc)]),
    "g53h_cache_slot_kind": (C.c_int, [C.POINTER(Glm53fExpertSrc)]),
    "g53h_set_speculate": (C.c_int, [C.c_int]),
    "g53h_speculate_counts": (None, [C.c_void_p]),
    "g53h_cache_layer_table": (C.c_int, [C.POINTER(Glm53fExpertSrc), C.c_int, C.POINTER(C.c_void_p),
                                         C.POINTER(C.c_void_p)]),
    "g53h_cache_init_store": (C.c_int, [C.POINTER(Glm53fCache), C.POINTER(G53hStore), C.POINTER(Glm53fCfg),
                                        C.c_int64, C.c_int, C.c_int]),
    "g53h_st_open": (C.c_int, [C.POINTER(Glm53fSt), C.c_char_p, C.c_int]),
    "g53h_st_close": (None, [C.POINTER(Glm53fSt)]),
    "g53h_st_index": (C.c_int, [C.POINTER(Glm53fSt), C.c_char_p]),
    "g53h_st_expert_bytes": (C.c_size_t, [C.POINTER(Glm53fCfg)]),
    "g53h_st_read_expert": (C.c_int, [C.POINTER(Glm53fSt), C.POINTER(Glm53fCfg), C.c_int, C.c_int, C.c_void_p,
                                      C.c_size_t, C.POINTER(Glm53fExpertQ)]),
    "g53h_store_synth_init": (C.c_int, [C.POINTER(G53hStore), C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                        C.c_uint64, C.c_float]),
    "g53h_store_synth_free": (None, [C.POINTER(G53hStore)]),
    "g53h_store_synth_key_scales": (C.c_int, [C.POINTER(G53hStore)]),
    "g53h_lru_trace": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int,
                                 C.c_void_p]),
}


def lib():
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise G53hError(f"{LIB_PATH} is not built; run __graft_entry__.build() or make -C "
                            f"{PKG_DIR}")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            if not hasattr(L, name):
                continue
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def exported_names():
    return sorted(_SIGS)


def check(rc, what=""):
    if rc != 0:
        raise G53hError(f"{what}: {lib().g53h_error().decode()}")


def init(device=0):
    L = lib()
    if L.g53h_device_count() < 1:
        raise G53hError("no HIP device visible; the MI355X path has no CPU fallback")
    check(L.g53h_init(device), "g53h_init")
    return L


def sync():
    check(lib().g53h_sync(), "g53h_sync")


# ----------------------------------------------------------------- device memory ----
class DevBuf:
    """A block of HBM owned by Python (freed when the object goes away)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = lib().g53h_alloc(max(self.nbytes, 1))
        if not self.ptr:
            raise G53hError(f"g53h_alloc({nbytes}): {lib().g53h_error().decode()}")

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().g53h_h2d(self.ptr, a.ctypes.data, a.nbytes), "g53h_h2d")

    def download(self, dtype, count=None, offset=0):
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype)
        check(lib().g53h_d2h(out.ctypes.data, self.ptr + offset, out.nbytes), "g53h_d2h")
        return out

    def zero(self):
        check(lib().g53h_memset(self.ptr, 0, self.nbytes), "g53h_memset")

    def free(self):
        if self.ptr and _lib is not None:
            _lib.g53h_free(self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def mem_info():
    f, t = C.c_size_t(), C.c_size_t()
    check(lib().g53h_mem_info(C.byref(f), C.byref(t)), "g53h_mem_info")
    return f.value, t.value
