"""GPU parity of the grouped path (batched decode and prefill, T >= 2): token-sorted grouped
GEMMs on the FP8 matrix cores, called through the C ABI (g53h_moe / g53h_moe_grouped).

Bar (the path's stated tolerance): routing indices and weights bit-exact; every output element
within 1e-2 absolute + 2e-3 relative of the reference's output for the same inputs. The
references are the C oracle (pinned to the compiled reference's outputs and golden vectors)
on CPU-sized cases, and the exact per-token GPU kernels (bit-exact with the oracle in
test_gpu_parity.py) at the full 2048-token size."""
import ctypes as C

import numpy as np
import pytest

import glm53h
import glm53h.synth as S
import oracle_lib as O
from glm53h import DevBuf, check

pytestmark = pytest.mark.gpu
ATOL, RTOL = 1e-2, 2e-3


def say(*a):
    print("[gpu]", *a, flush=True)


def within(got, want, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    err = np.abs(got - want)
    bound = ATOL + RTOL * np.abs(want)
    worst = float(np.max(err / bound)) if err.size else 0.0
    say(f"{what}: max |err| {err.max():.3e}, mean |err| {err.mean():.3e}, max |ref| {np.abs(want).max():.3f}, "
        f"worst err/bound {worst:.3f}")
    assert np.all(np.isfinite(got))
    assert np.all(err <= bound), what


@pytest.fixture(scope="module")
def L():
    return glm53h.init(0)


@pytest.fixture(scope="module")
def c2layer(L):
    say("building config-2 layer (288 experts in HBM)")
    return S.DeviceLayer.build(S.spec(2))


@pytest.fixture(scope="module")
def c3layer(L):
    say("building config-3 layer (Zipf-skewed bias)")
    return S.DeviceLayer.build(S.spec(3))


def run(layer, x, grouped, fn="g53h_moe"):
    sp, T = layer.sp, x.shape[0]
    L = glm53h.lib()
    prev = L.g53h_set_grouped(grouped)
    try:
        xd = DevBuf.from_array(x)
        out, idx, w = DevBuf(T * sp.E * 4), DevBuf(T * sp.K * 4), DevBuf(T * sp.K * 4)
        check(getattr(L, fn)(out.ptr, xd.ptr, T, C.byref(layer.layer), idx.ptr, w.ptr), fn)
        glm53h.sync()
        assert L.g53h_grouped_errors() == 0
    finally:
        L.g53h_set_grouped(prev)
    return (out.download(np.float32).reshape(T, sp.E), idx.download(np.int32).reshape(T, sp.K),
            w.download(np.float32).reshape(T, sp.K))


def oracle_out(layer, x, idx):
    sp = layer.sp
    mats = {int(e): layer.fetch_expert(int(e)) for e in np.unique(idx)}
    sh = layer.fetch_expert("shared") if sp.shared else None
    return O.moe(O.oracle(), x, sp, layer.router_f32, layer.bias_f32, mats, sh)


MID = dict(E=512, I=512, NE=16, K=8, router_sigma=0.02)


@pytest.mark.parametrize("T,shared", [(2, True), (33, True), (64, False), (300, True)])
def test_grouped_mid_shapes_vs_oracle(L, T, shared):
    """Hidden 512, inter 512, 16 experts top-8 (every expert gets ~T/2 tokens: several tiles per
    expert, partial tiles, tiles of one and of 33 positions), with and without the shared expert."""
    sp = S.LayerSpec(**MID, shared=shared)
    layer = S.DeviceLayer.build(sp)
    assert L.g53h_grouped_ok(C.byref(layer.layer)) == 1
    x = S.x_host(sp, T, batch=3)
    say("mid shapes T", T, "shared", shared)
    out, idx, w = run(layer, x, 1, "g53h_moe_grouped")
    want, wi, ww = oracle_out(layer, x, idx)
    assert np.array_equal(idx, wi) and np.array_equal(w.view(np.uint32), ww.view(np.uint32))
    within(out, want, f"mid T={T} shared={shared}")


def test_grouped_config3_batched_decode(L, c3layer):
    """64 tokens x top-8 over 288 Zipf-skewed experts. All 64 tokens against
    the exact GPU path, 6 of them against the oracle."""
    sp = c3layer.sp
    x = S.x_host(sp, 64, batch=0)
    say("config 3: grouped")
    out, idx, w = run(c3layer, x, 1)
    uniq = np.unique(idx)
    say("config 3: unique routed experts", len(uniq), "max tokens on one expert",
        int(np.bincount(idx.ravel()).max()))
    say("config 3: exact per-token path")
    ref, ri, rw = run(c3layer, x, 0)
    assert np.array_equal(idx, ri) and np.array_equal(w.view(np.uint32), rw.view(np.uint32))
    within(out, ref, "config 3 vs exact GPU path")
    sel = [0, 1, 17, 31, 50, 63]
    want, wi, _ = oracle_out(c3layer, x[sel], idx[sel])
    assert np.array_equal(idx[sel], wi)
    within(out[sel], want, "config 3 vs oracle")


def test_grouped_config4_prefill(L, c2layer):
    """2048 tokens, uniform routing (~57 tokens per expert), one planning
    pass. Against the exact GPU path on every token, and the oracle on 4 tokens."""
    sp = c2layer.sp
    T = 2048
    x = S.x_host(sp, T, batch=11)
    say("config 4: grouped, T", T)
    out, idx, w = run(c2layer, x, 1)
    say("config 4: exact per-token path")
    ref, ri, rw = run(c2layer, x, 0)
    assert np.array_equal(idx, ri) and np.array_equal(w.view(np.uint32), rw.view(np.uint32))
    within(out, ref, "config 4 vs exact GPU path")
    sel = [0, 1000, 2047]
    want, wi, _ = oracle_out(c2layer, x[sel], idx[sel])
    assert np.array_equal(idx[sel], wi)
    within(out[sel], want, "config 4 vs oracle")


def test_grouped_two_planning_passes(L, c2layer):
    """More tokens than one planning pass holds (2048 + 37): the second pass's outputs equal a
    separate call on those tokens bit for bit, and the whole call equals the exact path within
    the tolerance on a sample."""
    sp = c2layer.sp
    T = 2048 + 37
    x = S.x_host(sp, T, batch=12)
    say("two planning passes, T", T)
    out, idx, _ = run(c2layer, x, 1)
    tail, tidx, _ = run(c2layer, np.ascontiguousarray(x[2048:]), 1)
    assert np.array_equal(idx[2048:], tidx)
    assert np.array_equal(out[2048:].view(np.uint32), tail.view(np.uint32))
    ref, _, _ = run(c2layer, np.ascontiguousarray(x[2040:]), 0)
    within(out[2040:], ref, "two passes vs exact GPU path")


def test_grouped_is_deterministic(L, c2layer):
    sp = c2layer.sp
    x = S.x_host(sp, 96, batch=13)
    a, _, _ = run(c2layer, x, 1)
    b, _, _ = run(c2layer, x, 1)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_grouped_absent_expert_contributes_zero(L):
    """An expert whose descriptor has no weights (the reference's failed get: its slot
    contributes zero, src/core/glm53f_ops.c:1261-1270) gives the same output as the oracle with
    that expert's contributions zeroed."""
    sp = S.LayerSpec(**MID)
    layer = S.DeviceLayer.build(sp)
    x = S.x_host(sp, 40, batch=4)
    _, idx, _ = run(layer, x, 1, "g53h_moe_grouped")
    drop = int(idx[0, 0])
    descs = (S.G53hExpert * (sp.NE + 1))()
    C.memmove(descs, layer.experts, C.sizeof(descs))
    descs[drop].gate.w = None
    descs[drop].gate.flags = 1
    tab = DevBuf.from_array(np.frombuffer(bytes(descs), np.uint8))
    lay = S.G53hMoeLayer()
    C.memmove(C.byref(lay), C.byref(layer.layer), C.sizeof(lay))
    lay.experts = tab.ptr
    lay.shared = tab.ptr + sp.NE * C.sizeof(S.G53hExpert)
    L.g53h_set_grouped(1)
    xd = DevBuf.from_array(x)
    out = DevBuf(40 * sp.E * 4)
    check(L.g53h_moe_grouped(out.ptr, xd.ptr, 40, C.byref(lay), None, None), "grouped")
    glm53h.sync()
    assert L.g53h_grouped_errors() == 0
    got = out.download(np.float32).reshape(40, sp.E)
    mats = {int(e): layer.fetch_expert(int(e)) for e in np.unique(idx)}
    zero = [(np.zeros_like(w), np.zeros_like(s)) for w, s in mats[drop]]
    mats[drop] = zero                                  # zero codes and scales: contributions 0
    want, _, _ = O.moe(O.oracle(), x, sp, layer.router_f32, layer.bias_f32, mats, layer.fetch_expert("shared"))
    within(got, want, "absent expert")



def test_dropin_grouped_batches_vs_exact_and_oracle(L):
    """The C drop-in glm53f_moe at T >= 2 on grouped-eligible shapes (hidden 512, inter 512, 32
    experts top-8): the reference's protocol (get, compute and release the routed experts in
    batches, src/core/glm53f_ops.c:1240-1290) with the grouped kernels run once per batch and
    one combine at the end. Against the same call on the exact per-token kernels and the
    oracle, with and without the shared expert, with failing experts, and served from the HBM
    cache (bit-identical to the host-memory source: the plan does not depend on the batches)."""
    from test_gpu_cache import new_cache
    from test_gpu_parity import HostSrc, cfg_struct, dropin_moe, fmat

    sp = S.LayerSpec(**dict(MID, NE=32), shared=True)
    cf = cfg_struct(dict(E=sp.E, I=sp.I, NE=sp.NE, K=sp.K, routed_scale=sp.routed_scale, norm_topk=sp.norm_topk,
                         limit=sp.limit, br=sp.br, bc=sp.bc))
    W, b = S.router_host(sp), S.bias_host(sp)
    ex = {e: S.expert_host(sp, e) for e in range(sp.NE)}
    sh = S.expert_host(sp, "shared")
    T = 48
    x = S.x_host(sp, T, batch=5)

    def both(shared=True, drop=()):
        prev = L.g53h_set_grouped(1)
        try:
            src = HostSrc(cf, ex, drop)
            got = dropin_moe(cf, W, b, ex, sh, x, shared=shared, src=src)
            assert L.g53h_grouped_errors() == 0
            assert src.max_pinned <= sp.K and sorted(e for e in src.gets if e not in drop) == sorted(src.releases)
            assert len(set(src.gets)) > sp.K                 # more than one batch of experts
            L.g53h_set_grouped(0)
            ref = dropin_moe(cf, W, b, ex, sh, x, drop=drop, shared=shared)
        finally:
            L.g53h_set_grouped(prev)
        return got, ref

    say("drop-in grouped T", T, "with shared")
    got, ref = both()
    within(got, ref, "drop-in grouped vs exact")
    sel = [0, 7, 47]
    want, _, _ = O.moe(O.oracle(), x[sel], sp, W, b, ex, sh)
    within(got[sel], want, "drop-in grouped vs oracle")
    say("drop-in grouped, routed only")
    got_r, ref_r = both(shared=False)
    within(got_r, ref_r, "drop-in grouped routed-only vs exact")
    say("drop-in grouped, experts 3 and 20 failing")
    got_d, ref_d = both(drop=(3, 20))
    within(got_d, ref_d, "drop-in grouped with drops vs exact")
    assert not np.array_equal(got_d, got)

    say("drop-in grouped through the HBM cache")
    cf.n_layers = 2
    st = glm53h.G53hStore()
    check(L.g53h_store_synth_init(C.byref(st), sp.E, sp.I, 2, sp.NE, sp.NE, sp.seed, C.c_float(sp.expert_sigma)),
          "store")
    w = glm53h.Glm53fMoeW()
    w.gate, w.bias = W.ctypes.data, b.ctypes.data
    (gw, gs), (uw, us), (dw, ds) = sh
    w.sh_gate = fmat(gw, gs, sp.I, sp.E, sp.br, sp.bc)
    w.sh_up = fmat(uw, us, sp.I, sp.E, sp.br, sp.bc)
    w.sh_down = fmat(dw, ds, sp.E, sp.I, sp.br, sp.bc)
    try:
        for slots in (sp.K + 1, 40):
            c = new_cache(cf, st, slots, 0)
            prev = L.g53h_set_grouped(1)
            try:
                w.src = C.pointer(c.src)
                out = np.zeros((T, sp.E), np.float32)
                L.glm53f_moe(out.ctypes.data, x.ctypes.data, C.byref(w), C.byref(cf), T, None)
                assert L.g53h_grouped_errors() == 0
                say("cache slots", slots, "hits", c.hits, "misses", c.misses)
                assert np.array_equal(out.view(np.uint32), got.view(np.uint32))
            finally:
                L.g53h_set_grouped(prev)
                L.glm53f_cache_free(C.byref(c))
    finally:
        L.glm53f_forget_host_weights()
        L.g53h_store_synth_free(C.byref(st))
