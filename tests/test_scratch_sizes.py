"""The scratch sizes the reference's callers allocate by (glm53f_moe_scratch, glm53f_mlp_scratch,
src/core/glm53f_ops.c:991-1000, 496-500) equal the compiled reference's. No GPU: both are host
arithmetic."""
import ctypes as C

import pytest

import glm53h
import glm53h.synth as S
import oracle_lib as O


def cfg(sp):
    cf = glm53h.Glm53fCfg()
    cf.hidden, cf.moe_inter, cf.n_experts, cf.topk, cf.n_shared = sp.E, sp.I, sp.NE, sp.K, 1
    cf.routed_scale, cf.norm_topk, cf.swiglu_limit = sp.routed_scale, sp.norm_topk, sp.limit
    cf.fp8_block_r, cf.fp8_block_c = sp.br, sp.bc
    cf.dense_inter = 3 * sp.I
    return cf


@pytest.mark.skipif(not O.have_ref(), reason="reference not built")
def test_scratch_sizes_equal_the_reference():
    R = C.CDLL(O.REF_LIB)
    R.glm53f_moe_scratch.restype = C.c_size_t
    R.glm53f_mlp_scratch.restype = C.c_size_t
    for config in (1, 2):
        sp = S.spec(config)
        cf = cfg(sp)
        for T in (1, 5, 64, 65, 2048):
            assert glm53h.lib().glm53f_moe_scratch(C.byref(cf), T) == R.glm53f_moe_scratch(C.byref(cf), T), (config, T)
        assert glm53h.lib().glm53f_mlp_scratch(C.byref(cf)) == R.glm53f_mlp_scratch(C.byref(cf))
