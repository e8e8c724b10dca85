/* g53h_decode.hip - single-token decode of one MoE layer in two launches.
 *
 * The layer (reference src/core/glm53f_ops.c:1144-1342 at T = 1, with the router of
 * :945-976) is cut into work items of one 8 KB step of HBM codes for one wave:
 *
 *   R   one router row (bf16, 8 KB): the score of one expert
 *   G   one (gate row o, up row o) pair of one slot (2 x 4 KB of E4M3 codes) and its SwiGLU
 *   D   four down rows of one slot (4 x 2 KB of codes): four contributions
 *
 * Under a saturated HBM stream every access that crosses from one workgroup to another (an
 * atomic publish, a coherent poll) takes several microseconds, so the layer is arranged to
 * need almost none, and uses the kernel boundary (about 3 us) for the one dependency every
 * workgroup has: the routing.
 *
 * k_dec_route: the R items and the shared expert's G items, which depend on nothing, dealt
 *   over the grid. The last workgroup to finish (found by a counter after a release fence,
 *   when the GPU is nearly idle) selects the top-k of score + bias and writes the routing
 *   record: indices, weights, and the reference's outputs idx / w.
 *
 * k_dec_experts: every workgroup owns the same row groups of every slot's down product and a
 *   share of every slot's gate/up rows, so the final weighted combine is local to it. Its
 *   list runs: the shared expert's D items; then the routed slots' G items slot after slot,
 *   each slot's D items following two slots later (by then the slot's activation vector,
 *   written by all workgroups, is long complete); then the last slots' D items. Its four
 *   waves take items from the list through an LDS counter, one ahead: the codes of the next
 *   item are in flight while the current one is multiplied. Activations of the routed slots
 *   are published as 64-bit words carrying the launch's epoch in their upper half (by an
 *   atomic exchange, which is performed past the writer's L2); the first wave of a workgroup
 *   to claim a D item of a slot copies that vector into LDS with direct global->LDS loads
 *   issued with the item's codes, and checks the epochs when the item is multiplied (stale
 *   values are re-read). The buffers are never cleared: the epoch grows by one per launch.
 *
 * Arithmetic is the reference's, bit for bit (see g53h_gemv.h). Every wait is bounded: a wait
 * that runs out sets an error flag (read by g53h_decode_errors) and the wave goes on, so the
 * grid always drains. The grid is sized to the occupancy the runtime reports, so every
 * workgroup is resident at once.
 */
#include <hip/hip_runtime.h>
#include <math.h>

#include "g53h.h"
#include "g53h_core.h"
#include "g53h_gemv.h"
#include "g53h_kern.h"
#include "g53h_runtime.h"

#define G53_DEC_MAXK 15            /* top-k handled by the fused path (slots <= 16)      */
#define G53_DEC_MAXNE 1024
#define G53_DEC_E 4096
#define G53_DEC_I 2048
#define G53_DEC_NBE 32             /* 128-column blocks per gate/up row                  */
#define G53_DEC_NBI 16             /* 128-column blocks per down row                     */
#define G53_DEC_RPD 4              /* down rows per item                                 */
#define G53_DEC_NGRP (G53_DEC_E / G53_DEC_RPD)
#define G53_DEC_MAXRG 4            /* row groups one workgroup owns (grid >= 256)         */
#define G53_DEC_LAG 3              /* slots between a slot's G items and its D items      */
#define G53_DEC_NENT 3             /* activation copies a workgroup keeps in LDS          */
#define G53_DEC_ROT 16             /* copies of the tagged activations, used in rotation  */
#define G53_SPIN_LIMIT (1 << 20)   /* polls before a wait gives up                       */

typedef unsigned long long g53_u64;

/* ---------------------------------------------------------------- helpers ---- */
__device__ __forceinline__ g53_u64 g53_tag(unsigned epoch, float v)
{
    return ((g53_u64)epoch << 32) | __float_as_uint(v);
}
/* Publish a tagged value with an atomic exchange: a plain store, even an agent-scope one,
 * can stay in the writing XCD's L2 for tens of microseconds under load. */
__device__ __forceinline__ void g53_st_tag(g53_u64 *p, g53_u64 v)
{
    (void)__hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
/* Coherent reads (the sc1 cache policy: past this XCD's L2) through buffer loads. Unlike
 * atomic loads, which the compiler keeps in order, many of these can be in flight at once.
 * base must be uniform across the wave. */
__device__ __forceinline__ __amdgpu_buffer_rsrc_t g53_rsrc(const void *base)
{
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ g53_u64 g53_ld_coh64(__amdgpu_buffer_rsrc_t r, int byte_off)
{
    return __builtin_bit_cast(g53_u64, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, 16));
}
__device__ __forceinline__ float g53_ld_coh32f(__amdgpu_buffer_rsrc_t r, int byte_off)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 16));
}
__device__ __forceinline__ void g53_flag_err(int *err, int bit)
{
    __hip_atomic_fetch_or(err, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void g53_backoff() { __builtin_amdgcn_s_sleep(15); }   /* ~0.4 us */

/* LDS flags between the waves of one workgroup. LDS accesses of a workgroup are performed in
 * order, so relaxed accesses with a compiler barrier suffice; an acquire or release here would
 * also make the compiler wait for every outstanding global load, which would drain the
 * pipeline of codes in flight. */
#define G53_CBAR() asm volatile("" ::: "memory")
__device__ __forceinline__ int g53_lds_ld(int *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
__device__ __forceinline__ int g53_lds_add(int *p, int v)
{
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
/* Bounded sleep-poll of an LDS word until it is at least want. */
__device__ __forceinline__ bool g53_wait_lds(int *flag, int want)
{
    int spins = 0;
    while (g53_lds_ld(flag) < want) {
        if (++spins > 16 * G53_SPIN_LIMIT) return false;
        __builtin_amdgcn_s_sleep(2);
    }
    G53_CBAR();
    return true;
}

/* A descriptor the fused path can use: 128 x 128 blocks and the released shapes. */
__device__ __forceinline__ bool g53_desc_ok(const G53hExpert &e)
{
    return e.gate.br == 128 && e.gate.bc == 128 && e.gate.rows == G53_DEC_I && e.gate.cols == G53_DEC_E &&
           e.up.br == 128 && e.up.bc == 128 && e.up.rows == G53_DEC_I && e.up.cols == G53_DEC_E &&
           e.down.br == 128 && e.down.bc == 128 && e.down.rows == G53_DEC_E && e.down.cols == G53_DEC_I &&
           e.gate.scols >= G53_DEC_NBE && e.up.scols >= G53_DEC_NBE && e.down.scols >= G53_DEC_NBI;
}

/* Router dot product of one bf16 row (8 KB) whose 128 bytes for this lane are in c[], x in LDS
 * (padded blocks): columns lane*64 .. lane*64+63, every product exact in double, summed in
 * order per lane and then across the wave (the order of g53_router_dot). */
__device__ __forceinline__ double g53_router_row(const uint4 (&c)[8], const float *xs, int lane)
{
    double acc = 0.0;
    const uint32_t d[32] = {c[0].x, c[0].y, c[0].z, c[0].w, c[1].x, c[1].y, c[1].z, c[1].w,
                            c[2].x, c[2].y, c[2].z, c[2].w, c[3].x, c[3].y, c[3].z, c[3].w,
                            c[4].x, c[4].y, c[4].z, c[4].w, c[5].x, c[5].y, c[5].z, c[5].w,
                            c[6].x, c[6].y, c[6].z, c[6].w, c[7].x, c[7].y, c[7].z, c[7].w};
    const float *xl = xs + (lane >> 1) * G53_PADB + (lane & 1) * 64;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const float4 xq = *(const float4 *)(xl + 4 * k);
        acc += (double)g53_bitsf(d[2 * k] << 16) * (double)xq.x;
        acc += (double)g53_bitsf(d[2 * k] & 0xffff0000u) * (double)xq.y;
        acc += (double)g53_bitsf(d[2 * k + 1] << 16) * (double)xq.z;
        acc += (double)g53_bitsf(d[2 * k + 1] & 0xffff0000u) * (double)xq.w;
    }
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    return acc;
}

/* The sum, in lane order, of the doubles held by lanes base .. base+N-1 (base = lane rounded
 * down to a multiple of N), valid in lane base: the reference's sequential sum over a row's
 * blocks. The terms pass through pt, 64 doubles of LDS private to the wave. */
template <int N>
__device__ __forceinline__ double g53_row_sum(double t, double *pt, int lane)
{
    pt[lane] = t;
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    double s = 0.0;
    if ((lane & (N - 1)) == 0) {
#pragma unroll
        for (int k = 0; k < N; k += 2) {
            const double2 q = *(const double2 *)(pt + lane + k);
            s = s + q.x;
            s = s + q.y;
        }
    }
    __builtin_amdgcn_wave_barrier();
    return s;
}

/* One gate/up row pair (lanes 0-31 gate blocks, 32-63 up blocks) with x in LDS: the two row
 * sums in block order and the SwiGLU, valid in lane 0. */
__device__ __forceinline__ float g53_gateup_pair(const uint4 (&c)[8], float sc, const float *xs, double *pt,
                                                 float limit, const uint64_t *etab, int lane)
{
    const int bb = lane & 31;
    const double t = g53_blk_pad(c, xs + bb * G53_PADB) * (double)sc;
    const float v = (float)g53_row_sum<32>(t, pt, lane);
    const float u = __shfl(v, 32);
    return g53_swiglu1_tab(v, u, limit, etab);
}

extern "C" __device__ unsigned __ockl_wfred_max_u32(unsigned);
extern "C" __device__ unsigned __ockl_wfred_min_u32(unsigned);

/* Top-k of score + bias by one wave (reference src/core/glm53f_ops.c:957-969: K rounds of
 * "first strictly greater" arg-max, so the larger value first, the lower index among equal
 * values, NaN and -inf never), then the weights (:970-975). NV = ceil(NE / 64) values per lane;
 * each round is two wave reductions (the largest value, then the lowest index holding it).
 * The scores and biases are loaded by g53_topk_load first, so that other work can overlap the
 * loads. idx[j] = -1 where no expert could be selected (the reference aborts there; the return
 * value is then nonzero). */
template <int NV>
__device__ __forceinline__ void g53_topk_load(const float *score, const float *bias, int NE, float (&scv)[NV],
                                              float (&bl)[NV], int lane)
{
#pragma unroll
    for (int v = 0; v < NV; v++) {
        const int e = min(lane + 64 * v, NE - 1);
        scv[v] = score[e];
        bl[v] = bias[e];
    }
}

template <int NV>
__device__ __forceinline__ int g53_topk_weights(const float (&scv)[NV], const float (&bl)[NV], int NE, int K,
                                                int norm_topk, float routed_scale, int *idx, float *wv, int lane)
{
    uint32_t key[NV];
#pragma unroll
    for (int v = 0; v < NV; v++) {
        const float ch = scv[v] + bl[v];
        key[v] = (lane + 64 * v < NE && ch > -INFINITY) ? g53_fkey(ch) : 0u;    /* 0: never chosen */
    }
    int bad = 0;
    for (int j = 0; j < K; j++) {
        uint32_t m = 0;
        int mv = 0;
#pragma unroll
        for (int v = 0; v < NV; v++)
            if (key[v] > m) { m = key[v]; mv = v; }        /* strict: the lowest v among equals */
        const uint32_t g = __ockl_wfred_max_u32(m);
        if (g == 0) { bad = 1; if (lane == 0) { wv[j] = 0.0f; idx[j] = -1; } continue; }
        const uint32_t e = __ockl_wfred_min_u32(m == g ? (uint32_t)(lane + 64 * mv) : 0xffffffffu);
        if ((uint32_t)(lane + 64 * mv) == e && m == g) {  /* the owner of the winner */
            float sv = 0.0f;
#pragma unroll
            for (int v = 0; v < NV; v++)
                if (v == mv) { key[v] = 0; sv = scv[v]; }
            wv[j] = sv;
            idx[j] = (int)e;
        }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    /* the weights: every lane forms the sum in slot order, lane j divides weight j */
    float wj = 0.0f;
    if (lane < K) wj = wv[lane];
    if (norm_topk) {
        double s = 0.0;
        for (int j = 0; j < K; j++) s += (double)wv[j];
        if (lane < K) wj = (float)((double)wj / (s + 1e-20));
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    if (lane < K) wv[lane] = wj * routed_scale;
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    return bad;
}

/* Diagnostics: per-workgroup timestamps (100 MHz) into a.trace when it is set. */
#define G53_TRACE(k) do { if (a.trace && lane == 0) \
    a.trace[(size_t)blockIdx.x * 32 + (k)] = __builtin_amdgcn_s_memrealtime(); } while (0)

/* ------------------------------------------------------------ k_dec_route ---- */
struct G53RouteArgs {
    const float *x;
    const uint16_t *router;        /* bf16 [NE][E]                                       */
    float *score;                  /* [NE]                                               */
    int NE;
    g53_u64 *trace;                /* optional: [grid][32]; slots 9-10 of each workgroup  */
};

/* The router rows: one wave per row. */
__global__ void __launch_bounds__(64) k_dec_route(G53RouteArgs a)
{
    __shared__ __attribute__((aligned(16))) float xs[G53_DEC_NBE * G53_PADB];
    __shared__ uint64_t etab[32];                      /* the exponential's table */
    const int lane = threadIdx.x;
    G53_TRACE(9);
    for (int e = blockIdx.x; e < a.NE; e += gridDim.x) {
        uint4 c[8];
        g53_ld_blk(c, (const uint8_t *)(a.router + (size_t)e * G53_DEC_E + lane * 64));
        if (e == (int)blockIdx.x) {                    /* x into LDS while the row loads */
            if (lane < 32) etab[lane] = g53_exp2_tab_dev[lane];
            g53_vec_to_lds_pad<G53_DEC_E, 64>(xs, a.x, lane);
            __syncthreads();
        }
        const double d = g53_router_row(c, xs, lane);
        if (lane == 0) a.score[e] = g53_sigmoidf_tab((float)d, etab);
    }
    G53_TRACE(10);
}

/* ---------------------------------------------------------- k_dec_experts ---- */
struct G53ExpertsArgs {
    float *out;
    const float *x;
    const G53hExpert *experts;
    const G53hExpert *shared;
    const float *score;            /* [NE] written by k_dec_route                        */
    const float *bias;
    g53_u64 *act;                  /* [MAXK + 1][I] tagged activations, slot K = shared  */
    int *err;
    int *idx_out;                  /* the routing, written by workgroup 0 (may be NULL)   */
    float *w_out;
    int NE, K, norm_topk;
    unsigned epoch;
    float routed_scale, limit;
    g53_u64 *trace;                /* optional: [grid][32] timestamps and counters       */
};

enum { G53_IT_NONE = 0, G53_IT_G = 2, G53_IT_D = 3, G53_IT_A = 4 };

struct G53Item {
    int kind, s, r;                /* slot (K = the shared expert), and o / row group / half */
    int t;                         /* time slot (the order the slots are processed in)   */
};

/* The workgroup's list. Slots are processed in time order: the shared expert (when there is
 * one) first, then routed slots 0 .. K-1. With G_t = rows [g_lo, g_lo + g_n) of time slot t,
 * A_t = the two halves of its activation vector (copied into LDS), D_t = row groups [rg_lo,
 * rg_lo + n_rg) of its down product, L = G53_DEC_LAG:
 *   for t = 0 .. T-1:  [A_{t-L}] [G_t] [D_{t-L}]        then  [A_t][D_t] for t = T-L .. T-1
 * A slot's activations are read L slots after its G items were issued (so they are normally
 * complete), and a slot's A items come one G group ahead of its D items. */
struct G53List {
    int g_lo, g_n, rg_lo, n_rg, n, T;
};

__device__ __forceinline__ int g53_tslot(int t, int K, int has_shared)
{
    return has_shared ? (t == 0 ? K : t - 1) : t;
}

__device__ __forceinline__ G53Item g53_item(const G53List &l, int i, int K, int has_shared)
{
    G53Item it{G53_IT_NONE, 0, 0, 0};
    for (int t = 0; t < l.T; t++) {
        const int u = t - G53_DEC_LAG;
        if (u >= 0) {
            if (i < 2) { it.kind = G53_IT_A; it.t = u; it.s = g53_tslot(u, K, has_shared); it.r = i; return it; }
            i -= 2;
        }
        if (i < l.g_n) { it.kind = G53_IT_G; it.t = t; it.s = g53_tslot(t, K, has_shared); it.r = l.g_lo + i; return it; }
        i -= l.g_n;
        if (u >= 0) {
            if (i < l.n_rg) { it.kind = G53_IT_D; it.t = u; it.s = g53_tslot(u, K, has_shared); it.r = l.rg_lo + i; return it; }
            i -= l.n_rg;
        }
    }
    for (int u = l.T > G53_DEC_LAG ? l.T - G53_DEC_LAG : 0; u < l.T; u++) {
        if (i < 2) { it.kind = G53_IT_A; it.t = u; it.s = g53_tslot(u, K, has_shared); it.r = i; return it; }
        i -= 2;
        if (i < l.n_rg) { it.kind = G53_IT_D; it.t = u; it.s = g53_tslot(u, K, has_shared); it.r = l.rg_lo + i; return it; }
        i -= l.n_rg;
    }
    return it;
}

/* Addresses of one item's codes (this lane's 128 bytes) and block scale. Items that read
 * nothing point at the input vector instead, so that the loop issues its loads from one place
 * with no branch around them (a branch makes the compiler wait for the loads where the paths
 * join). Returns whether the item's codes are real. The matrices have 128 x 128 blocks, so
 * the scale row of output row r is r >> 7. */
__device__ __forceinline__ bool g53_addr(const G53Item &it, const G53hExpert *st, const g53_u64 *act,
                                         const float *dummy, int lane, const uint8_t *&p, const float *&ps)
{
    p = (const uint8_t *)dummy + lane * 128;
    ps = dummy;
    if (it.kind == G53_IT_A) {                /* 16 tagged activations per lane */
        p = (const uint8_t *)(act + (size_t)it.s * G53_DEC_I + it.r * 1024 + lane * 16);
        return true;
    }
    if (it.kind == G53_IT_G) {
        const G53hExpert &ex = st[it.s];
        if (!ex.gate.w) return false;
        const G53hMat &m = lane < 32 ? ex.gate : ex.up;
        const int b = lane & 31;
        p = m.w + (size_t)it.r * G53_DEC_E + b * 128;
        ps = m.s + (size_t)(it.r >> 7) * m.scols + b;
        return true;
    }
    if (it.kind == G53_IT_D) {
        const G53hExpert &ex = st[it.s];
        if (!ex.gate.w) return false;
        const G53hMat &m = ex.down;
        const int b = lane & 15, d = it.r * G53_DEC_RPD + (lane >> 4);
        p = m.w + (size_t)d * G53_DEC_I + b * 128;
        ps = m.s + (size_t)(d >> 7) * m.scols + b;
        return true;
    }
    return false;
}

__global__ void __launch_bounds__(256, 2) k_dec_experts(G53ExpertsArgs a)
{
    __shared__ __attribute__((aligned(16))) float xs[G53_DEC_NBE * G53_PADB];        /* padded x   */
    __shared__ __attribute__((aligned(16))) float actl[G53_DEC_NENT][G53_DEC_NBI * G53_PADB];
    __shared__ __attribute__((aligned(16))) double pw[4][64];                         /* row terms  */
    __shared__ G53hExpert st[G53_DEC_MAXK + 1];
    __shared__ float sw[16];
    __shared__ int sidx[16];
    __shared__ uint64_t etab[32];                      /* the exponential's table */
    __shared__ float cvals[G53_DEC_MAXRG][G53_DEC_RPD][G53_DEC_MAXK + 1];
    /* ent_ver[e]: activation halves copied into entry e so far; ent_used[e]: D items done with it */
    __shared__ int qctr, ndone, routed, ent_ver[G53_DEC_NENT], ent_used[G53_DEC_NENT];
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = a.K, hs = a.shared ? 1 : 0, nslots = K + hs;
    const int G = gridDim.x, b = blockIdx.x;

    G53List l;
    l.T = nslots;
    l.g_lo = (int)((long)G53_DEC_I * b / G);
    l.g_n = (int)((long)G53_DEC_I * (b + 1) / G) - l.g_lo;
    l.rg_lo = (int)((long)G53_DEC_NGRP * b / G);
    l.n_rg = (int)((long)G53_DEC_NGRP * (b + 1) / G) - l.rg_lo;
    l.n = nslots * (l.g_n + 2 + l.n_rg);
    const int ndone_all = nslots * l.n_rg;

    G53_TRACE(0);
    /* routing first, by wave 0: its loads go out before anything else */
    constexpr int NV = 5;                              /* scores per lane on the fast path */
    float scv[NV], bl[NV];
    const bool fast_route = a.NE <= 64 * NV;
    if (w == 0 && fast_route) g53_topk_load<NV>(a.score, a.bias, a.NE, scv, bl, lane);
    if (threadIdx.x < (int)(sizeof(G53hExpert) / 4) && a.shared)
        ((int *)&st[K])[threadIdx.x] = ((const int *)a.shared)[threadIdx.x];
    if (threadIdx.x == 0) { qctr = 0; ndone = 0; routed = 0; }
    if (threadIdx.x < 32) etab[threadIdx.x] = g53_exp2_tab_dev[threadIdx.x];
    if (threadIdx.x < G53_DEC_NENT) { ent_ver[threadIdx.x] = 0; ent_used[threadIdx.x] = 0; }
    g53_vec_to_lds_pad<G53_DEC_E, 256>(xs, a.x, threadIdx.x);
    __syncthreads();
    if (threadIdx.x == 0 && hs && st[K].gate.w && !g53_desc_ok(st[K])) {
        st[K].gate.w = nullptr;                        /* unusable: flagged, contributes zero */
        g53_flag_err(a.err, 8);
    }
    if (w == 0) {
        /* the routing: top-k, weights, the routed slots' descriptors; the other waves start on
         * the shared expert meanwhile */
        G53_TRACE(11);
        int bad;
        if (fast_route) {
            bad = g53_topk_weights<NV>(scv, bl, a.NE, K, a.norm_topk, a.routed_scale, sidx, sw, lane);
        } else {
            float sc16[G53_DEC_MAXNE / 64], b16[G53_DEC_MAXNE / 64];
            g53_topk_load<G53_DEC_MAXNE / 64>(a.score, a.bias, a.NE, sc16, b16, lane);
            bad = g53_topk_weights<G53_DEC_MAXNE / 64>(sc16, b16, a.NE, K, a.norm_topk, a.routed_scale, sidx, sw, lane);
        }
        if (bad && lane == 0) g53_flag_err(a.err, 2);
        G53_TRACE(13);
        if (b == 0 && lane < K) {
            if (a.idx_out) a.idx_out[lane] = sidx[lane];
            if (a.w_out) a.w_out[lane] = sw[lane];
        }
        const int words = (int)(sizeof(G53hExpert) / 4);
        for (int q = lane; q < K * words; q += 64) {
            const int j = q / words, ex = sidx[j];
            ((int *)st)[q] = (ex >= 0 && ex < a.NE) ? ((const int *)&a.experts[ex])[q % words] : 0;
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        if (lane < K && st[lane].gate.w && !g53_desc_ok(st[lane])) {
            st[lane].gate.w = nullptr;
            g53_flag_err(a.err, 8);
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        G53_CBAR();
        if (lane == 0) g53_lds_add(&routed, 1);
        G53_TRACE(14);
    }

    g53_u64 tw_act = 0, tw_comp = 0, n_items = 0, n_stale = 0, n_stale2 = 0;
    auto claim = [&]() -> int {
        int i = 0;
        if (lane == 0) i = g53_lds_add(&qctr, 1);
        return __builtin_amdgcn_readfirstlane(i);
    };

    /* multiply one item whose codes are in c[] */
    auto compute = [&](const G53Item &it, const uint4 (&c)[8], float sc, bool loaded) {
        if (it.kind == G53_IT_G) {
            if (!loaded) return;                             /* expert not there */
            const float v = g53_gateup_pair(c, sc, xs, pw[w], a.limit, etab, lane);
            if (lane == 0) g53_st_tag(a.act + (size_t)it.s * G53_DEC_I + it.r, g53_tag(a.epoch, v));
            return;
        }
        const int e = it.t % G53_DEC_NENT;
        if (it.kind == G53_IT_A) {
            /* half of slot s's activations: check the epochs (re-reading stale values) and
             * store the values into entry t % NENT once its previous slot is done with it */
            const int use = it.t / G53_DEC_NENT;
            if (!st[it.s].gate.w) {                          /* not used by any D item */
                G53_CBAR();
                if (lane == 0) g53_lds_add(&ent_ver[e], 1);
                return;
            }
            /* value 2k of this lane: c[k].x (value) / c[k].y (epoch); value 2k+1: c[k].z / c[k].w */
            uint32_t pending = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                if (c[k].y != a.epoch) pending |= 1u << (2 * k);
                if (c[k].w != a.epoch) pending |= 1u << (2 * k + 1);
            }
            if (use > 0 && !g53_wait_lds(&ent_used[e], use * l.n_rg) && lane == 0) g53_flag_err(a.err, 1);
            const int i0 = it.r * 1024 + lane * 16;          /* 16 values within one block */
            float *dst = actl[e] + (i0 >> 7) * G53_PADB + (i0 & 127);
#pragma unroll
            for (int k = 0; k < 4; k++)
                *(float4 *)(dst + 4 * k) = make_float4(__uint_as_float(c[2 * k].x), __uint_as_float(c[2 * k].z),
                                                       __uint_as_float(c[2 * k + 1].x), __uint_as_float(c[2 * k + 1].z));
            if (__ballot(pending != 0)) {
                /* stale values (read from a line this XCD's L2 took before they were written):
                 * re-read them coherently until their epochs are current, and store each back
                 * with a plain store, which refreshes the stale line for the workgroups of this
                 * XCD that read it later (the value stored is the one already in memory) */
                const g53_u64 t0 = __builtin_amdgcn_s_memrealtime();
                n_stale += __popc(pending);
                g53_u64 *src = a.act + (size_t)it.s * G53_DEC_I + it.r * 1024 + lane * 16;
                const __amdgpu_buffer_rsrc_t rsrc = g53_rsrc(a.act + (size_t)it.s * G53_DEC_I + it.r * 1024);
                int spins = 0;
                while (__ballot(pending != 0)) {
                    if (++spins > G53_SPIN_LIMIT) { if (lane == 0) g53_flag_err(a.err, 1); break; }
#pragma unroll
                    for (int h = 0; h < 16; h += 4) {
                        g53_u64 t[4];
#pragma unroll
                        for (int k = 0; k < 4; k++)
                            t[k] = (pending & (1u << (h + k))) ? g53_ld_coh64(rsrc, 8 * (lane * 16 + h + k)) : 0ull;
#pragma unroll
                        for (int k = 0; k < 4; k++)
                            if ((pending & (1u << (h + k))) && (unsigned)(t[k] >> 32) == a.epoch) {
                                dst[h + k] = __uint_as_float((uint32_t)t[k]);
                                src[h + k] = t[k];
                                pending &= ~(1u << (h + k));
                            }
                    }
                    if (spins == 1) n_stale2 += __popc(pending);
                    if (__ballot(pending != 0)) g53_backoff();
                }
                tw_act += __builtin_amdgcn_s_memrealtime() - t0;
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();
            G53_CBAR();
            if (lane == 0) g53_lds_add(&ent_ver[e], 1);
            return;
        }
        /* D item */
        float v = 0.0f;
        if (loaded) {
            const int want = 2 * (it.t / G53_DEC_NENT + 1);
            if (g53_lds_ld(&ent_ver[e]) < want) {
                const g53_u64 t0 = __builtin_amdgcn_s_memrealtime();
                if (!g53_wait_lds(&ent_ver[e], want) && lane == 0) g53_flag_err(a.err, 1);
                tw_act += __builtin_amdgcn_s_memrealtime() - t0;
            }
            const int bb = lane & 15;
            v = (float)g53_row_sum<16>(g53_blk_pad(c, actl[e] + bb * G53_PADB) * (double)sc, pw[w], lane);
        }
        if ((lane & 15) == 0) cvals[it.r - l.rg_lo][lane >> 4][it.s] = v;
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        G53_CBAR();
        int fin = 0;
        if (lane == 0) {
            g53_lds_add(&ent_used[e], 1);
            fin = g53_lds_add(&ndone, 1) == ndone_all - 1;
        }
        if (__builtin_amdgcn_readfirstlane(fin)) {
            /* every contribution of the workgroup's rows is in: combine them (reference
             * src/core/glm53f_ops.c:1329-1340) */
            G53_CBAR();
            const int m = lane >> 2, r = lane & 3;
            if (m < l.n_rg) {
                double acc = 0.0;
                for (int j = 0; j < K; j++) acc = acc + (double)sw[j] * (double)cvals[m][r][j];
                float o = (float)acc;
                if (hs) o = o + cvals[m][r][K];
                a.out[(l.rg_lo + m) * G53_DEC_RPD + r] = o;
            }
        }
    };

    /* ---- the item loop ----
     * Two code buffers alternate: each half-pass claims an item and issues its loads into the
     * free buffer (from one place, so the compiler keeps them in flight), then multiplies the
     * item in the other buffer. While a wave waits for one item's codes, the next item's are
     * already on their way. An item that needs the routing waits for it before its loads are
     * issued (wave 0 computes it while the others work on the shared expert). */
    uint4 ca[8], cb[8];
    float sa = 0.0f, sb = 0.0f;
    bool la, lb;
    auto next_item = [&]() -> G53Item {
        const int ni = claim();
        return ni < l.n ? g53_item(l, ni, K, hs) : G53Item{G53_IT_NONE, 0, 0, 0};
    };
    auto issue = [&](const G53Item &nt, uint4 (&c)[8], float &scv) -> bool {
        if ((nt.kind == G53_IT_G || nt.kind == G53_IT_D) && nt.s < K && g53_lds_ld(&routed) == 0) {
            if (!g53_wait_lds(&routed, 1) && lane == 0) g53_flag_err(a.err, 1);
        }
        const uint8_t *p;
        const float *ps;
        const bool r = g53_addr(nt, st, a.act, a.x, lane, p, ps);
        g53_ld_blk(c, p);
        scv = *(const g53_gf *)ps;
        return r;
    };
    auto run = [&](const G53Item &it, const uint4 (&c)[8], float scv, bool loaded) {
        const g53_u64 tc0 = __builtin_amdgcn_s_memrealtime();
        compute(it, c, scv, loaded);
        tw_comp += __builtin_amdgcn_s_memrealtime() - tc0;
        n_items++;
    };
    if (w == 0) G53_TRACE(8);
    G53Item ia = next_item(), ib;
    la = issue(ia, ca, sa);
    for (;;) {
        ib = next_item();
        lb = issue(ib, cb, sb);
        if (ia.kind == G53_IT_NONE) break;
        run(ia, ca, sa, la);
        ia = next_item();
        la = issue(ia, ca, sa);
        if (ib.kind == G53_IT_NONE) break;
        run(ib, cb, sb, lb);
    }
    G53_TRACE(2 + w);
    if (a.trace && lane == 0) {
        g53_u64 *tr = a.trace + (size_t)blockIdx.x * 32;
        tr[16 + w] = n_stale; tr[20 + w] = tw_act; tr[6] = n_stale2; tr[24 + w] = tw_comp; tr[28 + w] = n_items;
    }
}

/* ------------------------------------------------------------------ host side ---- */
static int g_dec_grid1 = -1;             /* workgroups of k_dec_experts, 0 = unavailable   */
static unsigned g_dec_epoch = 0;         /* epoch of the last launch                        */
static int *g_dec_state = nullptr;       /* [0] error flags                                 */
static void *g_dec_buf = nullptr;        /* scores | tagged activations                     */
static size_t g_dec_buf_bytes = 0;
static int g_dec_enabled = 1;
static g53_u64 *g_dec_trace = nullptr;

static int g53_dec_shape(const G53hMoeLayer *L)
{
    if (L->block_c != 128 || L->hidden != G53_DEC_E || L->inter != G53_DEC_I || L->router_dt != 1) return 0;
    if (L->topk < 1 || L->topk > G53_DEC_MAXK || L->n_experts > G53_DEC_MAXNE) return 0;
    return 1;
}

extern "C" int g53h_set_decode_trace(void *dev_buf)
{
    g_dec_trace = (g53_u64 *)dev_buf;
    return 0;
}

extern "C" int g53h_set_fused_decode(int on)
{
    const int old = g_dec_enabled;
    g_dec_enabled = on != 0;
    return old;
}

int g53h_decode_fused(float *out, const float *x, const G53hMoeLayer *L, int *idx_out, float *w_out)
{
    if (!g_dec_enabled || !g53_dec_shape(L)) return 1;     /* not handled: caller falls back */
    const int K = L->topk, NE = L->n_experts;
    const int cus = g53h_num_cus();
    if (g_dec_grid1 < 0) {
        int per = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, (const void *)k_dec_experts, 256, 0) != hipSuccess ||
            per < 1) {
            (void)hipGetLastError();
            g_dec_grid1 = 0;
        } else {
            g_dec_grid1 = (per > 2 ? 2 : per) * cus;
            /* every workgroup owns at most G53_DEC_MAXRG row groups */
            if ((G53_DEC_NGRP + g_dec_grid1 - 1) / g_dec_grid1 > G53_DEC_MAXRG) g_dec_grid1 = 0;
        }
        if (g_dec_grid1 && (hipMalloc((void **)&g_dec_state, 256) != hipSuccess ||
                            hipMemset(g_dec_state, 0, 256) != hipSuccess)) {
            (void)hipGetLastError();
            g_dec_grid1 = 0;
        }
    }
    if (!g_dec_grid1) return 1;
    /* scores [MAXNE] | tagged act [ROT][MAXK + 1][I], allocated and cleared once, so that no
     * tagged word carries a live epoch. The tagged activations rotate over ROT copies by
     * epoch, so a copy is reused only ROT launches later. */
    const size_t off_act = (size_t)G53_DEC_MAXNE * 4;
    const size_t act_copy = (size_t)(G53_DEC_MAXK + 1) * G53_DEC_I * 8;
    const size_t bytes = off_act + G53_DEC_ROT * act_copy;
    if (!g_dec_buf) {
        G53_TRY(hipMalloc(&g_dec_buf, bytes));
        G53_TRY(hipMemset(g_dec_buf, 0, bytes));
        G53_TRY(hipDeviceSynchronize());
        g_dec_buf_bytes = bytes;
        g_dec_epoch = 0;
    }
    if (++g_dec_epoch == 0) {                              /* wrapped: clear and start over */
        G53_TRY(hipStreamSynchronize(g53h_stream()));
        G53_TRY(hipMemset(g_dec_buf, 0, g_dec_buf_bytes));
        G53_TRY(hipDeviceSynchronize());
        g_dec_epoch = 1;
    }
    char *buf = (char *)g_dec_buf;
    G53RouteArgs r;
    r.x = x; r.router = (const uint16_t *)L->router; r.score = (float *)buf; r.NE = NE; r.trace = g_dec_trace;
    G53ExpertsArgs e;
    e.out = out; e.x = x; e.experts = L->experts; e.shared = L->shared;
    e.score = r.score; e.bias = L->bias;
    e.act = (g53_u64 *)(buf + off_act + (g_dec_epoch % G53_DEC_ROT) * act_copy);
    e.err = g_dec_state; e.idx_out = idx_out; e.w_out = w_out;
    e.NE = NE; e.K = K; e.norm_topk = L->norm_topk; e.epoch = g_dec_epoch;
    e.routed_scale = L->routed_scale; e.limit = L->swiglu_limit; e.trace = g_dec_trace;
    g53h_prof_mark(G53_PROF_START);
    hipLaunchKernelGGL(k_dec_route, dim3(NE), dim3(64), 0, g53h_stream(), r);
    G53_LAUNCHED("k_dec_route");
    g53h_prof_mark(G53_PROF_ROUTER);
    hipLaunchKernelGGL(k_dec_experts, dim3(g_dec_grid1), dim3(256), 0, g53h_stream(), e);
    G53_LAUNCHED("k_dec_experts");
    g53h_prof_mark(G53_PROF_FUSED);
    return 0;
}

extern "C" int g53h_decode_errors(void)
{
    if (g53h_ready() || !g_dec_state) return 0;
    int e = 0;
    if (hipStreamSynchronize(g53h_stream()) != hipSuccess) return -1;
    if (hipMemcpy(&e, g_dec_state, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess) return -1;
    if (e) (void)hipMemset(g_dec_state, 0, sizeof(int));
    return e;
}

extern "C" int g53h_decode_grid(void) { return g_dec_grid1; }
