/* g53h_xwg.h - device helpers for the one-launch decode kernels: values handed between the
 * workgroups of one launch (words tagged with the launch's epoch), coherent loads, bounded LDS
 * waits between the waves of a workgroup, the router row dot product and the top-k selection
 * by one wave. Included by g53h_decode.hip only. */
#ifndef G53H_XWG_H
#define G53H_XWG_H

#include <hip/hip_runtime.h>
#include <math.h>

#include "g53h.h"
#include "g53h_core.h"
#include "g53h_gemv.h"

#define G53_SPIN_LIMIT (1 << 20)   /* polls before a wait gives up                       */
#define G53_DEC_MAXK 15            /* top-k handled by the fused path (slots <= 16)      */
#define G53_DEC_MAXNE 1024
#define G53_DEC_E 4096             /* the released shapes the one-launch kernels take    */
#define G53_DEC_I 2048
#define G53_DEC_NBE 32             /* 128-column blocks per gate/up row                  */
#define G53_DEC_NBI 16             /* 128-column blocks per down row                     */

typedef unsigned long long g53_u64;
/* 16 bytes of codes in four VGPRs, as a native vector so that the compiler keeps each buffer
 * whole in registers */
typedef unsigned g53_u4 __attribute__((ext_vector_type(4)));

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
    return !((e.gate.flags | e.up.flags | e.down.flags) & G53H_MAT_I4) &&
           e.gate.br == 128 && e.gate.bc == 128 && e.gate.rows == G53_DEC_I && e.gate.cols == G53_DEC_E &&
           e.up.br == 128 && e.up.bc == 128 && e.up.rows == G53_DEC_I && e.up.cols == G53_DEC_E &&
           e.down.br == 128 && e.down.bc == 128 && e.down.rows == G53_DEC_E && e.down.cols == G53_DEC_I &&
           e.gate.scols >= G53_DEC_NBE && e.up.scols >= G53_DEC_NBE && e.down.scols >= G53_DEC_NBI;
}

/* Router dot product of one bf16 row (8 KB) whose 128 bytes for this lane are in c[], x read
 * from memory: columns lane*64 .. lane*64+63, every product exact in double, summed in
 * order per lane and then across the wave (the order of g53_router_dot). */
__device__ __forceinline__ double g53_router_row(const g53_u4 (&c)[8], const float *x, int lane)
{
    double acc = 0.0;
    const uint32_t d[32] = {c[0].x, c[0].y, c[0].z, c[0].w, c[1].x, c[1].y, c[1].z, c[1].w,
                            c[2].x, c[2].y, c[2].z, c[2].w, c[3].x, c[3].y, c[3].z, c[3].w,
                            c[4].x, c[4].y, c[4].z, c[4].w, c[5].x, c[5].y, c[5].z, c[5].w,
                            c[6].x, c[6].y, c[6].z, c[6].w, c[7].x, c[7].y, c[7].z, c[7].w};
    const float *xl = x + 64 * lane;                     /* this lane's 64 columns of x */
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


extern "C" __device__ unsigned __ockl_wfred_max_u32(unsigned);
#ifndef G53_RW_BREG
#define G53_RW_BREG 1
#endif

/* ------------------------------------------------------------------ routing ---- */
#ifndef G53_POLL_GAP
#define G53_POLL_GAP 8             /* s_sleep units (64 clocks) between two reads of the scores */
#endif
/* Top-k of score + bias by one wave (reference src/core/glm53f_ops.c:957-969: K rounds of
 * "first strictly greater" arg-max, so the larger value first, the lower index among equal
 * values, NaN and -inf never), then the weights (:970-975). The scores are the tagged words
 * other workgroups of this launch publish; they are read coherently, and re-read until every
 * tag carries this launch's epoch. Each lane sorts its keys; K rounds then take the wave
 * maximum of the lanes' first untaken keys (the lowest expert index among equal ones). sidx[j] = -1
 * where fewer than K experts are selectable (the reference aborts there; bit 2 of the error
 * flags is then set). Returns false when the scores did not all arrive in time. With nrouted
 * (an LDS counter), slot j is handed over as soon as its round ends: the counter reaches j + 1
 * once sidx[j] (and its pre-normalisation score in sw[j]) is written, and K at the end; the
 * normalised weights are final only when the function returns. With gbias, the selection's
 * code runs once on dummy values before anything is read (the instruction cache is warm when
 * the scores arrive), then the bias is copied from gbias into bias (LDS) and the scores read. */
template <int NV>
__device__ __forceinline__ bool g53_route_wave(const g53_u64 *score, const float *bias, int NE, int K, int norm_topk,
                                               float routed_scale, unsigned epoch, int *sidx, float *sw,
                                               uint32_t *kbuf, int *ebuf, int *err, int lane, g53_u64 &t_seen,
                                               int &n_polls, g53_u64 &t_tau, g53_u64 &t_rank, int limit,
                                               int *nrouted = nullptr, int *seenf = nullptr,
                                               const float *gbias = nullptr)
{
    const __amdgpu_buffer_rsrc_t rs = g53_rsrc(score);
    float scv[NV];
    uint32_t pend = (1u << NV) - 1;
    if (!gbias) {                                /* the first read: stale scores for pass 0 */
        pend = 0;
#pragma unroll
        for (int v = 0; v < NV; v++) {
            const int e = min(lane + 64 * v, NE - 1);
            const g53_u64 t = g53_ld_coh64(rs, 8 * e);
            scv[v] = __uint_as_float((uint32_t)t);
            if ((unsigned)(t >> 32) != epoch) pend |= 1u << v;
        }
    } else {
#pragma unroll
        for (int v = 0; v < NV; v++) scv[v] = 0.0f;
    }
    int spins = 0;
    int pos = 0;
    float bre[NV];                              /* the bias in registers (G53_RW_BREG) */
#pragma unroll
    for (int v = 0; v < NV; v++) bre[v] = 0.0f;
    /* two passes of the selection: the first on whatever the first read returned, while the
     * scores are still being computed (it runs the selection's code once, so that its
     * instructions are cached when the real pass runs), the second once every score is current */
#ifndef G53_RW_PASSES
#define G53_RW_PASSES 2
#endif
    constexpr int LAST = G53_RW_PASSES - 1;
#pragma clang loop unroll(disable)
    for (int pass = 0; pass < G53_RW_PASSES; pass++) {
    if (pass == 1) {
    if (gbias) {
        /* pass 0 ran first thing, on zeros and whatever the bias array held (only to bring the
         * selection's code into the instruction cache); now the bias, then the scores */
#if G53_RW_BREG
#pragma unroll
        for (int v = 0; v < NV; v++) bre[v] = gbias[min(lane + 64 * v, NE - 1)];
#else
        for (int e = lane; e < NE; e += 64) ((float *)bias)[e] = gbias[e];
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
#endif
    }
    /* two reads of the scores in flight at a time, issued a short sleep apart: a score that
     * lands is seen one memory latency later, not up to two */
    g53_u64 ta[NV], tb[NV];
    auto issue = [&](g53_u64 (&t)[NV]) {
#pragma unroll
        for (int v = 0; v < NV; v++) t[v] = g53_ld_coh64(rs, 8 * min(lane + 64 * v, NE - 1));
    };
    auto take = [&](const g53_u64 (&t)[NV]) {
#pragma unroll
        for (int v = 0; v < NV; v++)
            if ((pend & (1u << v)) && (unsigned)(t[v] >> 32) == epoch) {
                scv[v] = __uint_as_float((uint32_t)t[v]);
                pend &= ~(1u << v);
            }
        return __ballot(pend != 0) == 0;
    };
    if (__ballot(pend != 0)) {
        issue(ta);
        for (;;) {
            if (++spins > limit) return false;
            n_polls++;
            __builtin_amdgcn_s_sleep(G53_POLL_GAP);
            issue(tb);
            if (take(ta)) break;
            __builtin_amdgcn_s_sleep(G53_POLL_GAP);
            issue(ta);
            if (take(tb)) break;
        }
    }
    t_seen = __builtin_amdgcn_s_memrealtime();
    if (seenf && lane == 0) (void)g53_lds_add(seenf, 1);     /* every score is in */
    }
    uint32_t key[NV];
#pragma unroll
    for (int v = 0; v < NV; v++) {
        const int e = lane + 64 * v;
#if G53_RW_BREG
        const float ch = e < NE ? scv[v] + (gbias ? bre[v] : bias[e]) : -INFINITY;
#else
        const float ch = e < NE ? scv[v] + bias[e] : -INFINITY;
#endif
        key[v] = (ch > -INFINITY) ? g53_fkey(ch) : 0u;    /* 0: never chosen */
    }
    /* K rounds of arg-max. Each lane first sorts its keys, largest first and, among equal keys,
     * the lowest expert index first (a stable sort: the lane's experts are lane + 64 v in
     * increasing v). A round takes the wave maximum of the lanes' first keys; among lanes
     * holding it, the lowest expert index wins, and the winner shifts its list. */
    int vid[NV];
    float vsc[NV];
#pragma unroll
    for (int v = 0; v < NV; v++) { vid[v] = lane + 64 * v; vsc[v] = scv[v]; }
#pragma unroll
    for (int pass = 0; pass < NV; pass++)
#pragma unroll
        for (int q = pass & 1; q + 1 < NV; q += 2) {
            const bool sw_ = key[q + 1] > key[q];
            const uint32_t k0 = key[q], k1 = key[q + 1];
            const int i0 = vid[q], i1 = vid[q + 1];
            const float s0 = vsc[q], s1 = vsc[q + 1];
            key[q] = sw_ ? k1 : k0; key[q + 1] = sw_ ? k0 : k1;
            vid[q] = sw_ ? i1 : i0; vid[q + 1] = sw_ ? i0 : i1;
            vsc[q] = sw_ ? s1 : s0; vsc[q + 1] = sw_ ? s0 : s1;
        }
    if (pass == LAST) t_rank = __builtin_amdgcn_s_memrealtime();
    /* the lane's head: its first key not yet taken (index hp into the sorted list) */
    int hp = 0;
    uint32_t hk = key[0];
    int hv = vid[0];
    float hs = vsc[0];
    pos = 0;
    for (int j = 0; j < K; j++) {
        const uint32_t m = __ockl_wfred_max_u32(hk);
        if (m == 0) break;                                /* fewer than K selectable */
        const uint64_t cand = __ballot(hk == m);
        int win;
        if (__popcll(cand) == 1) win = (int)__builtin_ctzll(cand);
        else win = (int)(__ockl_wfred_min_u32(hk == m ? (uint32_t)hv : 0xffffffffu) & 63);
        const int e = __builtin_amdgcn_readlane(hv, win);
        const float wsc = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(hs), win));
        if (lane == 0) { sidx[j] = e; sw[j] = wsc; }
        if (pass == LAST && nrouted && lane == 0) { /* slot j is known: its tasks may start */
            G53_CBAR();
            (void)g53_lds_add(nrouted, 1);
        }
        hp += lane == win;                                /* the winner moves to its next key */
        hk = 0u;
#pragma unroll
        for (int q = 0; q < NV; q++)
            if (q == hp) { hk = key[q]; hv = vid[q]; hs = vsc[q]; }
        pos++;
    }
    }
    t_tau = __builtin_amdgcn_s_memrealtime();
    if (lane == 0)
        for (int j = pos; j < K; j++) { sidx[j] = -1; sw[j] = 0.0f; }
    if (nrouted && lane == 0 && pos < K) {
        G53_CBAR();
        (void)g53_lds_add(nrouted, K - pos);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    /* the weights: every lane forms the sum in slot order, lane j divides weight j */
    float wj = 0.0f;
    if (lane < K) wj = sw[lane];
    if (norm_topk) {
        double sum = 0.0;
        for (int q = 0; q < K; q++) sum += (double)sw[q];
        if (lane < K) wj = (float)((double)wj / (sum + 1e-20));
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    if (lane < K) sw[lane] = wj * routed_scale;
    if (pos < K && lane == 0) g53_flag_err(err, 2);
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    return true;
}

#endif /* G53H_XWG_H */
