/* g53h_moe.hip - the routed-expert MoE layer on gfx950.
 *
 * Decode path (bit-exact with the reference, src/core/glm53f_ops.c:1144-1342):
 *   1. router          k_router_scores + k_router_select_w (g53h_ops.hip)
 *   2. k_gateup        gate and up products of every slot (top-k experts + shared), SwiGLU
 *   3. k_down_combine  down product of every slot; the last workgroup to finish a row tile
 *                      combines the slots in double in top-k order and adds the shared expert
 *
 * The FP8 GEMV kernels read each expert's codes exactly once from HBM. A workgroup of 256
 * threads works in passes of 32 KB: every thread owns one 128-column block of one row per
 * pass, so the reference's lane structure (eight fp32 FMA chains of 16 steps, a double tree,
 * a double block scale, a double sum over blocks in order) is computed by one thread with no
 * cross-lane arithmetic, and the result is bit-identical to the CPU. The thread keeps the x
 * slice of its block (128 fp32) in registers for the whole workgroup. Codes are staged with
 * gfx950's direct global->LDS loads (global_load_lds_dwordx4): each wave instruction moves
 * 1 KB of consecutive HBM bytes, and the 16-byte chunks of a block are XOR-swizzled by the
 * block index so the threads' 128-byte reads do not collide on LDS banks. Two buffers let
 * the next pass stream in while the current one is multiplied.
 */
#include <hip/hip_runtime.h>
#include <math.h>

#include "g53h.h"
#include "g53h_core.h"
#include "g53h_kern.h"
#include "g53h_runtime.h"

typedef float g53_f2 __attribute__((ext_vector_type(2)));

#include "g53h_gemv.h"

/* Work is spread over the whole GPU in grid-stride order: at step j, wave w takes chunk
 * j * nwaves + w, so the waves running together read one contiguous sweep of HBM (regularly
 * strided per-wave ranges make many waves hit the same HBM channels at once). A chunk is 64
 * lanes x one 128-column block = 8 KB of consecutive codes per matrix stream. Each lane writes
 * its block's scaled double term to LDS; after its last step every lane takes one buffered
 * row and adds its terms in block order (the reference's sequential double sum). */

/* Gate and up products with the SwiGLU. A chunk is OPS = 32/NBLK consecutive values of o of
 * one slot; lane l of a step holds block l % NBLK of row l / NBLK, rows alternating gate o,
 * up o, gate o+1, up o+1, ... Dynamic LDS: x (swizzled), the slot table, and the term buffer
 * of 4 waves x steps*64/NBLK rows. Grid: (nwaves / 4, T), 256 threads. */
template <int NBLK>
__global__ void __launch_bounds__(256, 2)
k_gateup(float *__restrict__ act, const float *__restrict__ x, int E, int I, int nslots,
         const G53hExpert *__restrict__ slots, float limit, int nwaves, int steps)
{
    constexpr int RPW = 64 / NBLK, OPS = RPW / 2, PST = NBLK + 1;
    extern __shared__ __attribute__((aligned(16))) double dyn_gu[];
    float *xs = (float *)dyn_gu;                              /* NBLK*128 floats        */
    G53hExpert *st = (G53hExpert *)(xs + NBLK * 128);         /* nslots descriptors     */
    double *pball = (double *)(st + nslots);                  /* [4][steps*RPW*PST]     */
    const int t = blockIdx.y;
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wave = blockIdx.x * 4 + w;
    const int b = lane % NBLK, rw = lane / NBLK, ol = rw >> 1, up = rw & 1;
    const int cps = I / OPS, total = nslots * cps;            /* chunks per slot, chunks */
    {
        const int words = nslots * (int)(sizeof(G53hExpert) / 4);
        const int *src = (const int *)(slots + (size_t)t * nslots);
        for (int q = threadIdx.x; q < words; q += 256) ((int *)st)[q] = src[q];
    }
    g53_vec_to_lds(xs, x + (size_t)t * E, E, threadIdx.x, 256);
    __syncthreads();
    const float *xb = xs + b * 128;
    double *pw = pball + (size_t)w * steps * RPW * PST;
    uint4 cur[8];
    float sc = 0.0f;
    int c = wave;
    bool have = c < total && st[c / cps].gate.w != nullptr;
    if (have) {
        const int s = c / cps, o = (c % cps) * OPS + ol;
        const G53hMat &m = up ? st[s].up : st[s].gate;
        g53_ld_blk(cur, m.w + (size_t)o * E + b * 128);
        sc = ((g53_gf *)m.s)[(size_t)(o / m.br) * m.scols + b];
    }
    for (int j = 0; j < steps; j++, c += nwaves) {
        const int cn = c + nwaves;
        const bool hn = j + 1 < steps && cn < total && st[cn / cps].gate.w != nullptr;
        uint4 nxt[8];
        float scn = 0.0f;
        if (hn) {
            const int s = cn / cps, o = (cn % cps) * OPS + ol;
            const G53hMat &m = up ? st[s].up : st[s].gate;
            g53_ld_blk(nxt, m.w + (size_t)o * E + b * 128);
            scn = ((g53_gf *)m.s)[(size_t)(o / m.br) * m.scols + b];
        }
        if (have) pw[(j * RPW + rw) * PST + b] = g53_blk_lds(cur, xb, b) * (double)sc;
        have = hn;
        sc = scn;
#pragma unroll
        for (int k = 0; k < 8; k++) cur[k] = nxt[k];
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);                      /* lgkmcnt(0): the term writes */
    __builtin_amdgcn_wave_barrier();
    /* lane r sums buffered row r: step r / RPW, row r % RPW of that step */
    const int jr = lane / RPW, rr = lane % RPW, cr = wave + jr * nwaves;
    const bool mine = lane < steps * RPW && cr < total && st[cr / cps].gate.w != nullptr;
    float v = 0.0f;
    if (mine) {
        double accd = 0.0;
        const double *pr = pw + lane * PST;
        for (int bb = 0; bb < NBLK; bb++) accd = accd + pr[bb];
        v = (float)accd;
    }
    const float u = __shfl_down(v, 1);                        /* up row of the same o */
    if (mine && !(rr & 1)) {
        const int s = cr / cps, o = (cr % cps) * OPS + (rr >> 1);
        act[((size_t)t * nslots + s) * I + o] = g53_swiglu1(v, u, limit);
    }
}

/* Down products: contrib[t][s][d] = (down_s act[t][s])[d] for the present slots (zeros for a
 * dropped expert, nothing for an absent one). A chunk is RPW = 64/NBLK consecutive rows of one
 * slot. Every slot's activation sits in LDS (swizzled). Dynamic LDS: activations, the slot
 * table, the term buffer of nw waves x steps*RPW rows. Grid: (nwaves / nw, T), 64*nw threads. */
template <int NBLK>
__global__ void __launch_bounds__(1024)
k_down(float *__restrict__ contrib, const float *__restrict__ act, int E, int I, int nslots,
       const G53hExpert *__restrict__ slots, int nwaves, int steps)
{
    constexpr int RPW = 64 / NBLK, PST = NBLK + 1;
    extern __shared__ __attribute__((aligned(16))) double dyn_dn[];
    const int nw = blockDim.x >> 6, nthr = blockDim.x;
    float *as = (float *)dyn_dn;                              /* [nslots][I]            */
    G53hExpert *st = (G53hExpert *)(as + (size_t)nslots * I);
    double *pball = (double *)(st + nslots);                  /* [nw][steps*RPW*PST]    */
    const int t = blockIdx.y;
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wave = blockIdx.x * nw + w;
    const int b = lane % NBLK, rw = lane / NBLK;
    const int cps = E / RPW, total = nslots * cps;
    {
        const int words = nslots * (int)(sizeof(G53hExpert) / 4);
        const int *src = (const int *)(slots + (size_t)t * nslots);
        for (int q = threadIdx.x; q < words; q += nthr) ((int *)st)[q] = src[q];
    }
    for (int sl = 0; sl < nslots; sl++)
        g53_vec_to_lds(as + (size_t)sl * I, act + ((size_t)t * nslots + sl) * I, I, threadIdx.x, nthr);
    __syncthreads();
    double *pw = pball + (size_t)w * steps * RPW * PST;
    uint4 cur[8];
    float sc = 0.0f;
    int c = wave;
    bool have = c < total && st[c / cps].gate.w != nullptr;
    if (have) {
        const G53hMat &m = st[c / cps].down;
        const int d = (c % cps) * RPW + rw;
        g53_ld_blk(cur, m.w + (size_t)d * I + b * 128);
        sc = ((g53_gf *)m.s)[(size_t)(d / m.br) * m.scols + b];
    }
    for (int j = 0; j < steps; j++, c += nwaves) {
        const int cn = c + nwaves;
        const bool hn = j + 1 < steps && cn < total && st[cn / cps].gate.w != nullptr;
        uint4 nxt[8];
        float scn = 0.0f;
        if (hn) {
            const G53hMat &m = st[cn / cps].down;
            const int d = (cn % cps) * RPW + rw;
            g53_ld_blk(nxt, m.w + (size_t)d * I + b * 128);
            scn = ((g53_gf *)m.s)[(size_t)(d / m.br) * m.scols + b];
        }
        if (have) pw[(j * RPW + rw) * PST + b] = g53_blk_lds(cur, as + (size_t)(c / cps) * I + b * 128, b) * (double)sc;
        have = hn;
        sc = scn;
#pragma unroll
        for (int k = 0; k < 8; k++) cur[k] = nxt[k];
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    const int jr = lane / RPW, rr = lane % RPW, cr = wave + jr * nwaves;
    if (lane < steps * RPW && cr < total) {
        const int s = cr / cps, d = (cr % cps) * RPW + rr;
        if (st[s].gate.w) {
            double accd = 0.0;
            const double *pr = pw + lane * PST;
            for (int bb = 0; bb < NBLK; bb++) accd = accd + pr[bb];
            contrib[((size_t)t * nslots + s) * E + d] = (float)accd;
        } else if ((st[s].gate.flags & G53H_MAT_DROPPED)) {
            contrib[((size_t)t * nslots + s) * E + d] = 0.0f;
        }
    }
}

/* Generic combine for the fallback path (any shape): contrib [T][nslots][E]. */
__global__ void k_combine(float *__restrict__ out, const float *__restrict__ contrib,
                          const float *__restrict__ wts, int T, int E, int K, int nslots)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)T * E) return;
    const int t = (int)(i / E), d = (int)(i % E);
    const float *ct = contrib + (size_t)t * nslots * E;
    double acc = 0.0;
    for (int j = 0; j < K; j++) acc = acc + (double)wts[(size_t)t * K + j] * (double)ct[(size_t)j * E + d];
    float o = (float)acc;
    if (nslots > K) o = o + ct[(size_t)K * E + d];
    out[i] = o;
}

/* ------------------------------------------------------------------ dispatch ---- */
/* Allow a kernel more than the default 64 KB of dynamic LDS (gfx950 has 160 KB per CU). */
static int g53_lds_attr(const void *fn, size_t bytes)
{
    if (bytes <= 65536) return 0;
    G53_TRY(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
    return 0;
}

static int g53_pow2_le(int v, int lim) { return v >= 1 && v <= lim && (v & (v - 1)) == 0; }

/* The block-lane kernels need 128-column blocks and 2 to 32 blocks per row of gate/up and 1
 * to 32 per row of down (powers of two), whole chunks of rows, at most 64 slots and every
 * slot's activation within LDS. */
static int g53_fast_ok(const G53hMoeLayer *L)
{
    const int E = L->hidden, I = L->inter, nslots = L->topk + (L->shared ? 1 : 0);
    if (L->block_c != 128 || E % 128 || I % 128 || nslots > 64) return 0;
    const int nbe = E / 128, nbi = I / 128;
    if (!g53_pow2_le(nbe, 32) || nbe < 2 || !g53_pow2_le(nbi, 32)) return 0;
    if ((size_t)nslots * I * 4 > 100 * 1024) return 0;
    return I % (32 / nbe) == 0 && E % (64 / nbi) == 0;
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

/* fused != 0: every slot's expert is present or dropped, and the layer output is combined in
 * the same launch. fused == 0: contributions of the present slots only go to contrib (slots
 * whose descriptor is absent are left as they are), for the caller to combine later. */
static int g53_layer_body(float *out, const float *x, int T, const G53hMoeLayer *L, const int *idx,
                          const float *wts, char *ws, float *contrib, int fused, const G53hExpert *slots)
{
    const int E = L->hidden, I = L->inter, K = L->topk;
    const int nslots = K + (L->shared ? 1 : 0);
    float *act = (float *)ws;
    hipStream_t st = g53h_stream();
    if (g53_fast_ok(L)) {
        const int nbe = E / 128, nbi = I / 128;
        const int rpw_e = 64 / nbe, rpw_i = 64 / nbi, cus = g53h_num_cus();
        /* gate/up: about 8 waves per CU in grid-stride order; each wave buffers at most 64 rows */
        const int tot_gu = nslots * (I / (rpw_e / 2));
        int nw_gu = 8 * cus;
        if (nw_gu > tot_gu) nw_gu = tot_gu;
        int st_gu = (tot_gu + nw_gu - 1) / nw_gu;
        while (st_gu * rpw_e > 64) { nw_gu *= 2; st_gu = (tot_gu + nw_gu - 1) / nw_gu; }
        nw_gu = (nw_gu + 3) / 4 * 4;
        const size_t lds1 = (size_t)nbe * 128 * 4 + (size_t)nslots * sizeof(G53hExpert) +
                            (size_t)4 * st_gu * rpw_e * (nbe + 1) * 8;
        /* down: one workgroup of 16 waves per CU, every slot's activation in its LDS */
        const int tot_dn = nslots * (E / rpw_i);
        int wpg = 16, nw_dn = wpg * cus;
        if (nw_dn > tot_dn) { nw_dn = (tot_dn + wpg - 1) / wpg * wpg; }
        int st_dn = (tot_dn + nw_dn - 1) / nw_dn;
        while (st_dn * rpw_i > 64) { nw_dn *= 2; st_dn = (tot_dn + nw_dn - 1) / nw_dn; }
        const size_t lds2 = (size_t)nslots * I * 4 + (size_t)nslots * sizeof(G53hExpert) +
                            (size_t)wpg * st_dn * rpw_i * (nbi + 1) * 8;
        if (lds2 > 160 * 1024) return g53h_fail("g53h_moe: %zu bytes of LDS for the down kernel", lds2);
        dim3 g1(nw_gu / 4, T), g2(nw_dn / wpg, T);
#define G53_GU(N) case N: if (g53_lds_attr((const void *)k_gateup<N>, lds1)) return -1; \
                          hipLaunchKernelGGL(k_gateup<N>, g1, dim3(256), lds1, st, act, x, E, I, nslots, slots, \
                                             L->swiglu_limit, nw_gu, st_gu); break
#define G53_DN(N) case N: if (g53_lds_attr((const void *)k_down<N>, lds2)) return -1; \
                          hipLaunchKernelGGL(k_down<N>, g2, dim3(64 * wpg), lds2, st, contrib, act, E, I, nslots, \
                                             slots, nw_dn, st_dn); break
        switch (nbe) { G53_GU(2); G53_GU(4); G53_GU(8); G53_GU(16); G53_GU(32); }
        G53_LAUNCHED("k_gateup");
        g53h_prof_mark(G53_PROF_GATEUP);
        switch (nbi) { G53_DN(1); G53_DN(2); G53_DN(4); G53_DN(8); G53_DN(16); G53_DN(32); }
        G53_LAUNCHED("k_down");
        g53h_prof_mark(G53_PROF_DOWN);
#undef G53_GU
#undef G53_DN
        if (!fused) return 0;
        if (g53h_combine_into(out, contrib, wts, T, E, K, nslots)) return -1;
        g53h_prof_mark(G53_PROF_COMBINE);
        return 0;
    }
    /* int4 experts and any other shape: the row-wave kernels, same arithmetic */
    if (g53h_rows_layer(contrib, act, x, T, nslots, slots, E, I, L->swiglu_limit)) return -1;
    g53h_prof_mark(G53_PROF_GENERIC);
    if (!fused) return 0;
    return g53h_combine_into(out, contrib, wts, T, E, K, nslots);
}

int g53h_combine_into(float *out, const float *contrib, const float *wts, int T, int E, int K, int nslots)
{
    const long n = (long)T * E;
    hipLaunchKernelGGL(k_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, g53h_stream(), out,
                       contrib, wts, T, E, K, nslots);
    G53_LAUNCHED("k_combine");
    return 0;
}

static size_t g53_layer_ws_bytes(const G53hMoeLayer *L, int T)
{
    const int I = L->inter, K = L->topk, nslots = K + (L->shared ? 1 : 0);
    return align256((size_t)T * nslots * I * 4) + align256((size_t)2 * T * nslots * I * 4);
}

static size_t g53_contrib_bytes(const G53hMoeLayer *L, int T)
{
    return align256((size_t)T * (L->topk + (L->shared ? 1 : 0)) * L->hidden * 4);
}

static size_t g53_slots_bytes(const G53hMoeLayer *L, int T)
{
    return align256((size_t)T * (L->topk + (L->shared ? 1 : 0)) * sizeof(G53hExpert));
}

static int g53_check_layer(const G53hMoeLayer *L, int T)
{
    if (!L) return g53h_fail("g53h_moe: no layer");
    if (T < 0) return g53h_fail("g53h_moe: T %d", T);
    if (L->hidden <= 0 || L->inter <= 0) return g53h_fail("g53h_moe: hidden %d inter %d", L->hidden, L->inter);
    if (L->topk < 1 || L->topk > GLM53F_MAX_TOPK_DEV || L->topk > L->n_experts)
        return g53h_fail("g53h_moe: topk %d of %d experts", L->topk, L->n_experts);
    if (!L->experts) return g53h_fail("g53h_moe: no expert table");
    return 0;
}

/* Octet-tiled experts are read by the single-token decode kernel k_dec_tiled (released
 * shapes) and the grouped kernels (T >= 2 where the grouped path takes the layer), MFMA-tiled
 * ones by k_dec_mfma only; the per-token kernels of this file assume row-major codes, so any
 * other case is refused. */
static int g53_tiled_refused(const char *fn, int T)
{
    return g53h_fail("%s: tiled experts are read only by the single-token decode kernels (T = 1, hidden %d, "
                     "inter %d, 128x128 blocks, top-k <= 15, bf16 router or given routing) and the grouped kernels "
                     "(T >= 2, grouped path on, octet-tiled only); this call has T = %d", fn, 4096, 2048, T);
}

extern "C" int g53h_moe_routed_given(float *out, const float *x, int T, const G53hMoeLayer *L,
                                     const int *idx, const float *wts)
{
    if (g53h_ready() || g53_check_layer(L, T)) return -1;
    if (T == 0) return 0;
    if (T == 1 && L->tiled) {                    /* one launch that skips the routing */
        const int r = (L->tiled == 2 || L->tiled == 4) ? g53h_decode_mtiled(out, x, L, nullptr, nullptr, idx, wts)
                                    : g53h_decode_tiled(out, x, L, nullptr, nullptr, idx, wts);
        if (r <= 0) return r;
    }
    if (L->tiled) return g53_tiled_refused("g53h_moe_routed_given", T);
    const size_t ssz = g53_slots_bytes(L, T), csz = g53_contrib_bytes(L, T);
    char *ws = (char *)g53h_workspace(ssz + csz + g53_layer_ws_bytes(L, T));
    if (!ws) return -1;
    G53hExpert *slots = (G53hExpert *)ws;
    if (g53h_resolve_slots(slots, L->experts, idx, L->shared, T, L->topk)) return -1;
    return g53_layer_body(out, x, T, L, idx, wts, ws + ssz + csz, (float *)(ws + ssz), 1, slots);
}

extern "C" int g53h_moe_partial(float *contrib, const float *x, int T, const G53hMoeLayer *L,
                                const int *idx)
{
    if (g53h_ready() || g53_check_layer(L, T)) return -1;
    if (T == 0) return 0;
    if (L->tiled) return g53_tiled_refused("g53h_moe_partial", T);
    const size_t ssz = g53_slots_bytes(L, T);
    char *ws = (char *)g53h_workspace(ssz + g53_layer_ws_bytes(L, T));
    if (!ws) return -1;
    G53hExpert *slots = (G53hExpert *)ws;
    if (g53h_resolve_slots(slots, L->experts, idx, L->shared, T, L->topk)) return -1;
    return g53_layer_body(nullptr, x, T, L, idx, nullptr, ws + ssz, contrib, 0, slots);
}

extern "C" int g53h_moe_combine(float *out, const float *contrib, const float *wts, int T,
                                const G53hMoeLayer *L)
{
    if (g53h_ready() || g53_check_layer(L, T)) return -1;
    if (T == 0) return 0;
    return g53h_combine_into(out, contrib, wts, T, L->hidden, L->topk, L->topk + (L->shared ? 1 : 0));
}

extern "C" int g53h_moe(float *out, const float *x, int T, const G53hMoeLayer *L, int *idx_out,
                        float *w_out)
{
    if (g53h_ready() || g53_check_layer(L, T)) return -1;
    if (T == 0) return 0;
    if (!L->router || !L->bias) return g53h_fail("g53h_moe: no router");
    if (T == 1) {                                    /* single-token decode: one fused launch */
        const int r = (L->tiled == 2 || L->tiled == 4) ? g53h_decode_mtiled(out, x, L, idx_out, w_out, nullptr, nullptr)
                      : L->tiled  ? g53h_decode_tiled(out, x, L, idx_out, w_out, nullptr, nullptr)
                                  : g53h_decode_fused(out, x, L, idx_out, w_out);
        if (r <= 0) return r;
    }
    if (g53h_grouped_use(L, T)) return g53h_moe_grouped(out, x, T, L, idx_out, w_out);
    if (L->tiled) return g53_tiled_refused("g53h_moe", T);
    const int K = L->topk, NE = L->n_experts;
    const size_t rsz = align256((size_t)2 * T * NE * 4), isz = align256((size_t)T * K * 4);
    const size_t ssz = g53_slots_bytes(L, T), csz = g53_contrib_bytes(L, T);
    char *ws = (char *)g53h_workspace(rsz + 2 * isz + ssz + csz + g53_layer_ws_bytes(L, T));
    if (!ws) return -1;
    int *idx = idx_out ? idx_out : (int *)(ws + rsz);
    float *w = w_out ? w_out : (float *)(ws + rsz + isz);
    G53hExpert *slots = (G53hExpert *)(ws + rsz + 2 * isz);
    g53h_prof_mark(G53_PROF_START);
    if (g53h_router_into(idx, w, x, T, L->router, L->router_dt, L->bias, NE, L->hidden, K, L->norm_topk,
                         L->routed_scale, nullptr, (float *)ws, L->experts, L->shared, slots))
        return -1;
    g53h_prof_mark(G53_PROF_ROUTER);
    return g53_layer_body(out, x, T, L, idx, w, ws + rsz + 2 * isz + ssz + csz,
                          (float *)(ws + rsz + 2 * isz + ssz), 1, slots);
}
