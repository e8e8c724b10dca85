/* g53h_moe.hip - the routed-expert MoE layer on gfx950.
 *
 * Decode path (bit-exact with the reference, src/core/glm53f_ops.c:1144-1342):
 *   1. router          k_router_scores + k_router_select (g53h_ops.hip)
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

#define G53_WG 256
#define G53_PASS (G53_WG * 128)        /* bytes of codes per pass: one block per thread */
#define G53_MAXPASS 4                  /* passes per workgroup */

typedef float g53_f2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void *g53_lds_ptr;

/* One 16-byte direct HBM->LDS load per lane (global_load_lds_dwordx4): lane i's bytes land at
 * LDS offset lds_base + 16*i. Issued as inline assembly so that the compiler's wait-count
 * pass does not treat every LDS read as dependent on every pending copy (it then waits for
 * all of them and the double buffer never overlaps); the kernels wait explicitly with
 * g53_wait_vm_keep8 / g53_wait_vm_all and publish with g53_barrier. M0 carries the LDS base;
 * nothing else in these kernels uses M0. */
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void g53_dma16(const void *src, uint32_t lds_base)
{
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(src), "s"(lds_base) : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t g53_lds_addr(const void *p)
{
    return (uint32_t)(uintptr_t)(g53_lds_ptr)p;
}

/* Stage one pass of codes into LDS. The pass is RP rows of NBLK*128 bytes; row lr of the
 * pass starts at rowptr(lr). Chunk c (16 B) of the pass lands at LDS offset 16*c and holds
 * block b = (c/8) % NBLK, 16-byte piece k = (c%8) ^ (b&7) of row lr = c / (8*NBLK). Each wave
 * instruction covers 64 consecutive chunks, i.e. 1 KB of consecutive HBM bytes. */
template <int NBLK, typename RowPtr>
__device__ __forceinline__ void g53_stage(uint8_t *lds, RowPtr rowptr)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t base = g53_lds_addr(lds);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int ci = (wave * 8 + i) * 64;          /* first chunk of this wave instruction */
        const int c = ci + lane;
        const int lr = c / (8 * NBLK);
        const int b = (c >> 3) % NBLK;
        const int k = (c & 7) ^ (b & 7);
        const uint8_t *src = rowptr(lr) + b * 128 + k * 16;
        g53_dma16(src, __builtin_amdgcn_readfirstlane(base + (uint32_t)ci * 16));
    }
}

/* Workgroup barrier that publishes LDS writes, without the compiler's fence (which would also
 * drain the in-flight HBM->LDS copies of the next pass). */
__device__ __forceinline__ void g53_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

/* The reference's block sum for the thread's (row, block): codes from LDS, x from registers. */
template <int NBLK>
__device__ __forceinline__ double g53_block_sum(const uint8_t *lds, int lr, int b, const float (&xr)[128])
{
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const uint8_t *base = lds + (size_t)(lr * NBLK + b) * 128;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint4 q = *(const uint4 *)(base + 16 * (k ^ (b & 7)));
        const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int h = 0; h < 2; h++) {                /* column step 2k + h, columns 16k+8h+l */
            const g53_f2 w0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)d[2 * h], false);
            const g53_f2 w1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)d[2 * h], true);
            const g53_f2 w2 = __builtin_amdgcn_cvt_pk_f32_fp8((int)d[2 * h + 1], false);
            const g53_f2 w3 = __builtin_amdgcn_cvt_pk_f32_fp8((int)d[2 * h + 1], true);
            const int e = 16 * k + 8 * h;
            a[0] = __builtin_fmaf(w0[0], xr[e + 0], a[0]);
            a[1] = __builtin_fmaf(w0[1], xr[e + 1], a[1]);
            a[2] = __builtin_fmaf(w1[0], xr[e + 2], a[2]);
            a[3] = __builtin_fmaf(w1[1], xr[e + 3], a[3]);
            a[4] = __builtin_fmaf(w2[0], xr[e + 4], a[4]);
            a[5] = __builtin_fmaf(w2[1], xr[e + 5], a[5]);
            a[6] = __builtin_fmaf(w3[0], xr[e + 6], a[6]);
            a[7] = __builtin_fmaf(w3[1], xr[e + 7], a[7]);
        }
    }
    return (((double)a[0] + a[4]) + ((double)a[2] + a[6]))
         + (((double)a[1] + a[5]) + ((double)a[3] + a[7]));
}

__device__ __forceinline__ void g53_load_x(float (&xr)[128], const float *x)
{
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const float4 v = *(const float4 *)(x + 4 * i);
        xr[4 * i + 0] = v.x; xr[4 * i + 1] = v.y; xr[4 * i + 2] = v.z; xr[4 * i + 3] = v.w;
    }
}

__device__ __forceinline__ void g53_wait_vm_keep8() { asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); }
__device__ __forceinline__ void g53_wait_vm_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ const G53hExpert *g53_slot_expert(const G53hExpert *experts, const int *idx,
                                                             const G53hExpert *shared, int K, int t, int s)
{
    return s < K ? &experts[idx[(size_t)t * K + s]] : shared;
}

/* act[t][s][o] = swiglu(gate_s x_t, up_s x_t) for o in this workgroup's rows.
 * Grid: (I / (HALF*npass), nslots, T); HALF = RP/2 rows of gate and of up per pass. */
template <int NBLK>
__global__ void __launch_bounds__(G53_WG, 2)
k_gateup(float *__restrict__ act, const float *__restrict__ x, int E, int I, int K, int nslots,
         const G53hExpert *__restrict__ experts, const int *__restrict__ idx,
         const G53hExpert *__restrict__ shared, int npass, float limit)
{
    constexpr int RP = G53_WG / NBLK, HALF = RP / 2;
    __shared__ __attribute__((aligned(16))) uint8_t codes[2][G53_PASS];
    __shared__ double pbuf[2][G53_WG];
    __shared__ float sct[G53_MAXPASS][G53_WG];
    const int s = blockIdx.y, t = blockIdx.z;
    const G53hExpert *ex = g53_slot_expert(experts, idx, shared, K, t, s);
    const uint8_t *gw = ex->gate.w, *uw = ex->up.w;
    if (!gw) return;                                   /* dropped expert: down writes zeros */
    const float *gs = ex->gate.s, *us = ex->up.s;
    const int br = ex->gate.br, scols = ex->gate.scols;
    const int tid = threadIdx.x, lr = tid / NBLK, b = tid % NBLK;
    const int o_first = blockIdx.x * HALF * npass;

    float xr[128];
    g53_load_x(xr, x + (size_t)t * E + b * 128);

    auto rowptr_of = [&](int p) {
        return [=](int r) -> const uint8_t * {
            const int o = o_first + p * HALF + (r < HALF ? r : r - HALF);
            return (r < HALF ? gw : uw) + (size_t)o * E;
        };
    };
    for (int p = 0; p < npass; p++) {                 /* this thread's block scales, per pass */
        const int o = o_first + p * HALF + (lr < HALF ? lr : lr - HALF);
        sct[p][tid] = (lr < HALF ? gs : us)[(size_t)(o / br) * scols + b];
    }
    g53_stage<NBLK>(codes[0], rowptr_of(0));
#pragma unroll 1
    for (int p = 0; p < npass; p++) {
        const int cur = p & 1;
        if (p + 1 < npass) {
            g53_stage<NBLK>(codes[cur ^ 1], rowptr_of(p + 1));
            g53_wait_vm_keep8();
        } else {
            g53_wait_vm_all();
        }
        const float sc = sct[p][tid];
        g53_barrier();
        const double bs = g53_block_sum<NBLK>(codes[cur], lr, b, xr);
        pbuf[cur][tid] = bs * (double)sc;
        g53_barrier();
        if (tid < HALF) {
            double ag = 0.0, au = 0.0;
#pragma unroll 4
            for (int j = 0; j < NBLK; j++) ag = ag + pbuf[cur][tid * NBLK + j];
#pragma unroll 4
            for (int j = 0; j < NBLK; j++) au = au + pbuf[cur][(tid + HALF) * NBLK + j];
            const int oo = o_first + p * HALF + tid;
            act[((size_t)t * nslots + s) * I + oo] = g53_swiglu1((float)ag, (float)au, limit);
        }
    }
}

/* contrib[t][s][d] = down_s act[t][s] for this workgroup's rows; the last of the nslots
 * workgroups of a row tile then writes out[t][d] = (float)(sum_j w_j * contrib_j[d]) (+ the
 * shared slot). Grid: (E / (RP*npass), nslots, T). */
template <int NBLK>
__global__ void __launch_bounds__(G53_WG, 2)
k_down_combine(float *__restrict__ out, float *__restrict__ contrib, const float *__restrict__ act,
               int E, int I, int K, int nslots, const G53hExpert *__restrict__ experts,
               const int *__restrict__ idx, const float *__restrict__ wts,
               const G53hExpert *__restrict__ shared, int npass, int *__restrict__ counters, int fused)
{
    constexpr int RP = G53_WG / NBLK;
    __shared__ __attribute__((aligned(16))) uint8_t codes[2][G53_PASS];
    __shared__ double pbuf[2][G53_WG];
    __shared__ float sct[G53_MAXPASS][G53_WG];
    __shared__ int last;
    const int s = blockIdx.y, t = blockIdx.z;
    const G53hExpert *ex = g53_slot_expert(experts, idx, shared, K, t, s);
    const uint8_t *dw = ex->down.w;
    const int tid = threadIdx.x, lr = tid / NBLK, b = tid % NBLK;
    const int d_first = blockIdx.x * RP * npass, rows = RP * npass;
    float *crow = contrib + ((size_t)t * nslots + s) * E;

    if (dw && ex->gate.w) {
        const float *ds = ex->down.s;
        const int br = ex->down.br, scols = ex->down.scols;
        float xr[128];
        g53_load_x(xr, act + ((size_t)t * nslots + s) * I + b * 128);
        auto rowptr_of = [&](int p) {
            return [=](int r) -> const uint8_t * { return dw + (size_t)(d_first + p * RP + r) * I; };
        };
        for (int p = 0; p < npass; p++)
            sct[p][tid] = ds[(size_t)((d_first + p * RP + lr) / br) * scols + b];
        g53_stage<NBLK>(codes[0], rowptr_of(0));
#pragma unroll 1
        for (int p = 0; p < npass; p++) {
            const int cur = p & 1;
            if (p + 1 < npass) {
                g53_stage<NBLK>(codes[cur ^ 1], rowptr_of(p + 1));
                g53_wait_vm_keep8();
            } else {
                g53_wait_vm_all();
            }
            const float sc = sct[p][tid];
            g53_barrier();
            const double bs = g53_block_sum<NBLK>(codes[cur], lr, b, xr);
            pbuf[cur][tid] = bs * (double)sc;
            g53_barrier();
            if (tid < RP) {
                double acc = 0.0;
#pragma unroll 4
                for (int j = 0; j < NBLK; j++) acc = acc + pbuf[cur][tid * NBLK + j];
                crow[d_first + p * RP + tid] = (float)acc;
            }
        }
    } else if (ex->gate.pad_ == G53_DROPPED) {
        for (int r = tid; r < rows; r += G53_WG) crow[d_first + r] = 0.0f;
    }
    if (!fused) return;

    /* arrival: publish this slot's rows, and let the last slot of the tile combine */
    __threadfence();
    __syncthreads();
    int *cnt = counters + (size_t)t * gridDim.x + blockIdx.x;
    if (tid == 0) last = (atomicAdd(cnt, 1) == nslots - 1);
    __syncthreads();
    if (!last) return;
    __threadfence();
    const float *wt = wts + (size_t)t * K;
    const float *ct = contrib + (size_t)t * nslots * E;
    for (int r = tid; r < rows; r += G53_WG) {
        const int d = d_first + r;
        double acc = 0.0;
        for (int j = 0; j < K; j++) {
            const float c = __builtin_nontemporal_load(ct + (size_t)j * E + d);
            acc = acc + (double)wt[j] * (double)c;
        }
        float o = (float)acc;
        if (nslots > K) o = o + __builtin_nontemporal_load(ct + (size_t)K * E + d);
        out[(size_t)t * E + d] = o;
    }
    if (tid == 0) *cnt = 0;
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
static int g53_pow2_le(int v, int lim) { return v >= 1 && v <= lim && (v & (v - 1)) == 0; }

/* The tiled kernels need 128-column blocks, column counts that are powers of two multiples
 * of 128, and row counts that fill whole passes. */
static int g53_fast_ok(const G53hMoeLayer *L, int *np_gu, int *np_dn)
{
    const int E = L->hidden, I = L->inter;
    if (L->block_c != 128 || E % 128 || I % 128) return 0;
    const int nbe = E / 128, nbi = I / 128;
    if (!g53_pow2_le(nbe, 128) || !g53_pow2_le(nbi, 128)) return 0;
    const int half = (G53_WG / nbe) / 2, rp = G53_WG / nbi;
    if (half < 1 || I % half || E % rp) return 0;
    int a = I / half, c = E / rp;                     /* passes per slot */
    int pg = G53_MAXPASS, pd = G53_MAXPASS;
    while (pg > 1 && a % pg) pg >>= 1;
    while (pd > 1 && c % pd) pd >>= 1;
    *np_gu = pg;
    *np_dn = pd;
    return 1;
}

/* Expert descriptors must describe 128x128-block FP8 matrices of the layer's shape for the
 * tiled path; the host drop-in checks this per expert, g53h_moe trusts the caller. */
static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

int g53h_router_into(int *idx, float *w, const float *x, int T, const void *gate, int dt,
                     const float *bias, int NE, int E, int K, int norm_topk, float scale,
                     int *nan_flag, float *scratch);

/* fused != 0: every slot's expert is present or dropped, and the layer output is combined in
 * the same launch. fused == 0: contributions of the present slots only go to contrib (slots
 * whose descriptor is absent are left as they are), for the caller to combine later. */
static int g53_layer_body(float *out, const float *x, int T, const G53hMoeLayer *L, const int *idx,
                          const float *wts, char *ws, float *contrib, int fused)
{
    const int E = L->hidden, I = L->inter, K = L->topk;
    const int nslots = K + (L->shared ? 1 : 0);
    float *act = (float *)ws;
    hipStream_t st = g53h_stream();
    int np_gu = 0, np_dn = 0;
    if (g53_fast_ok(L, &np_gu, &np_dn)) {
        const int nbe = E / 128, nbi = I / 128;
        const int half = (G53_WG / nbe) / 2, rp = G53_WG / nbi;
        const int tiles = E / (rp * np_dn);
        int *counters = g53h_counters();
        if ((long)T * tiles > 4096) return g53h_fail("g53h_moe: %d tokens x %d tiles exceed the counters", T, tiles);
        dim3 g1(I / (half * np_gu), nslots, T), g2(tiles, nslots, T);
#define G53_GU(N) case N: hipLaunchKernelGGL(k_gateup<N>, g1, dim3(G53_WG), 0, st, act, x, E, I, K, nslots, \
                                             L->experts, idx, L->shared, np_gu, L->swiglu_limit); break
#define G53_DN(N) case N: hipLaunchKernelGGL(k_down_combine<N>, g2, dim3(G53_WG), 0, st, out, contrib, act, E, I, \
                                             K, nslots, L->experts, idx, wts, L->shared, np_dn, counters, fused); break
        switch (nbe) { G53_GU(1); G53_GU(2); G53_GU(4); G53_GU(8); G53_GU(16); G53_GU(32); G53_GU(64); G53_GU(128); }
        G53_LAUNCHED("k_gateup");
        g53h_prof_mark(G53_PROF_GATEUP);
        switch (nbi) { G53_DN(1); G53_DN(2); G53_DN(4); G53_DN(8); G53_DN(16); G53_DN(32); G53_DN(64); G53_DN(128); }
        G53_LAUNCHED("k_down_combine");
        g53h_prof_mark(G53_PROF_DOWN);
#undef G53_GU
#undef G53_DN
        return 0;
    }
    /* any other shape: one thread per (token, slot, row), same arithmetic */
    float *g = (float *)(ws + align256((size_t)T * nslots * I * sizeof(float)));
    float *u = g + (size_t)T * nslots * I;
    if (g53h_slot_mm_generic(g, x, T, K, nslots, L->experts, idx, L->shared, 0, I, E, 0)) return -1;
    if (g53h_slot_mm_generic(u, x, T, K, nslots, L->experts, idx, L->shared, 1, I, E, 0)) return -1;
    if (g53h_swiglu_split(act, g, u, (long)T * nslots * I, L->swiglu_limit)) return -1;
    if (g53h_slot_mm_generic(contrib, act, T, K, nslots, L->experts, idx, L->shared, 2, E, I, 1)) return -1;
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
    const int E = L->hidden, I = L->inter, K = L->topk, nslots = K + (L->shared ? 1 : 0);
    (void)E;
    return align256((size_t)T * nslots * I * 4) + align256((size_t)2 * T * nslots * I * 4);
}

static size_t g53_contrib_bytes(const G53hMoeLayer *L, int T)
{
    return align256((size_t)T * (L->topk + (L->shared ? 1 : 0)) * L->hidden * 4);
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

extern "C" int g53h_moe_routed_given(float *out, const float *x, int T, const G53hMoeLayer *L,
                                     const int *idx, const float *wts)
{
    if (g53h_ready() || g53_check_layer(L, T)) return -1;
    if (T == 0) return 0;
    char *ws = (char *)g53h_workspace(g53_contrib_bytes(L, T) + g53_layer_ws_bytes(L, T));
    if (!ws) return -1;
    return g53_layer_body(out, x, T, L, idx, wts, ws + g53_contrib_bytes(L, T), (float *)ws, 1);
}

extern "C" int g53h_moe_partial(float *contrib, const float *x, int T, const G53hMoeLayer *L,
                                const int *idx)
{
    if (g53h_ready() || g53_check_layer(L, T)) return -1;
    if (T == 0) return 0;
    char *ws = (char *)g53h_workspace(g53_layer_ws_bytes(L, T));
    if (!ws) return -1;
    return g53_layer_body(nullptr, x, T, L, idx, nullptr, ws, contrib, 0);
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
    const int K = L->topk, NE = L->n_experts;
    const size_t rsz = align256((size_t)2 * T * NE * 4), isz = align256((size_t)T * K * 4);
    const size_t csz = g53_contrib_bytes(L, T);
    char *ws = (char *)g53h_workspace(rsz + 2 * isz + csz + g53_layer_ws_bytes(L, T));
    if (!ws) return -1;
    int *idx = idx_out ? idx_out : (int *)(ws + rsz);
    float *w = w_out ? w_out : (float *)(ws + rsz + isz);
    g53h_prof_mark(G53_PROF_START);
    if (g53h_router_into(idx, w, x, T, L->router, L->router_dt, L->bias, NE, L->hidden, K, L->norm_topk,
                         L->routed_scale, nullptr, (float *)ws))
        return -1;
    g53h_prof_mark(G53_PROF_ROUTER);
    return g53_layer_body(out, x, T, L, idx, w, ws + rsz + 2 * isz + csz, (float *)(ws + rsz + 2 * isz), 1);
}
