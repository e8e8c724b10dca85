/* g53h_gemv.h - device building blocks of the bit-exact FP8 GEMV kernels (decode path). */
#ifndef G53H_GEMV_H
#define G53H_GEMV_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "g53h.h"
#include "g53h_core.h"

/* Block-lane layout. Lane i of a wave owns 128-column block i % NBLK of row i / NBLK, so one
 * wave instruction reads 64 consecutive 16-byte pieces spaced 128 bytes apart, and the eight
 * loads of a block cover 64 * 128 consecutive bytes of HBM: a wave streams 8 KB of contiguous
 * codes per step. Every lane computes the reference's sum of its block (eight fp32 FMA chains
 * over columns l, l+8, ..., the double tree, times the block scale) and writes that double
 * to LDS; the row's double sum over blocks, which the reference takes in block order, is then
 * formed by one lane per row reading the row's terms in order. */
typedef float g53_f2 __attribute__((ext_vector_type(2)));

/* Expert pointers come from a descriptor in memory, so the compiler cannot tell they are
 * global and would emit flat loads, which also count against the LDS wait counter. Loads
 * through the global address space keep the two counters apart. */
#if defined(__HIP_DEVICE_COMPILE__)
typedef __attribute__((address_space(1))) const uint4 g53_gu4;
typedef __attribute__((address_space(1))) const float g53_gf;
#else
typedef const uint4 g53_gu4;
typedef const float g53_gf;
#endif

__device__ __forceinline__ void g53_ld_blk(uint4 (&c)[8], const uint8_t *p)
{
    g53_gu4 *q = (g53_gu4 *)p;
#pragma unroll
    for (int k = 0; k < 8; k++) c[k] = q[k];
}

/* The block sum with x in LDS, stored swizzled: 16-byte chunk q of block b sits at chunk
 * q ^ (b & 31) of the block, so the lanes of different blocks read different banks. */
__device__ __forceinline__ double g53_blk_lds(const uint4 (&c)[8], const float *xb, int b)
{
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t d[4] = {c[k].x, c[k].y, c[k].z, c[k].w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = 4 * k + i, e = 4 * q, l = e & 7;
            const float4 xq = *(const float4 *)(xb + 4 * (q ^ (b & 31)));
            const g53_f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)d[i], false);
            const g53_f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)d[i], true);
            a[l + 0] = __builtin_fmaf(lo[0], xq.x, a[l + 0]);
            a[l + 1] = __builtin_fmaf(lo[1], xq.y, a[l + 1]);
            a[l + 2] = __builtin_fmaf(hi[0], xq.z, a[l + 2]);
            a[l + 3] = __builtin_fmaf(hi[1], xq.w, a[l + 3]);
        }
    }
    return (((double)a[0] + a[4]) + ((double)a[2] + a[6]))
         + (((double)a[1] + a[5]) + ((double)a[3] + a[7]));
}

/* Padded block layout: 128-column block b of a vector starts at float b * G53_PADB, so that
 * the 8 lanes of one ds_read_b128 phase, each reading chunk q of a different block, hit
 * different LDS banks, and a lane's 32 chunk reads are one base address plus immediate
 * offsets. */
#define G53_PADB 132

template <class V>
__device__ __forceinline__ double g53_blk_pad(const V (&c)[8], const float *xb)
{
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t d[4] = {c[k].x, c[k].y, c[k].z, c[k].w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = 4 * k + i, e = 4 * q, l = e & 7;
            const float4 xq = *(const float4 *)(xb + 4 * q);
            const g53_f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)d[i], false);
            const g53_f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)d[i], true);
            a[l + 0] = __builtin_fmaf(lo[0], xq.x, a[l + 0]);
            a[l + 1] = __builtin_fmaf(lo[1], xq.y, a[l + 1]);
            a[l + 2] = __builtin_fmaf(hi[0], xq.z, a[l + 2]);
            a[l + 3] = __builtin_fmaf(hi[1], xq.w, a[l + 3]);
        }
    }
    return (((double)a[0] + a[4]) + ((double)a[2] + a[6]))
         + (((double)a[1] + a[5]) + ((double)a[3] + a[7]));
}

/* Copy a vector of N floats (N a multiple of 4 * NTHR) into LDS in the padded block layout,
 * every load issued before the first store. */
template <int N, int NTHR>
__device__ __forceinline__ void g53_vec_to_lds_pad(float *dst, const float *src, int tid)
{
    constexpr int PER = N / 4 / NTHR;
    float4 v[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) v[k] = *(const float4 *)(src + 4 * (tid + k * NTHR));
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int e = 4 * (tid + k * NTHR);
        *(float4 *)(dst + (e / 128) * G53_PADB + (e % 128)) = v[k];
    }
}

/* Copy a vector of n floats (n a multiple of 128) into LDS with the block swizzle. */
__device__ __forceinline__ void g53_vec_to_lds(float *dst, const float *src, int n, int tid, int nthr)
{
    for (int c = tid; c < n / 4; c += nthr) {
        const int e = 4 * c, blk = e / 128, q = (e % 128) / 4;
        *(float4 *)(dst + blk * 128 + 4 * (q ^ (blk & 31))) = *(const float4 *)(src + e);
    }
}

/* Gate and up products with the SwiGLU. Wave w of the grid owns n_o consecutive values of o of
 * one slot: it streams the n_o gate rows (RPW = 64/NBLK rows per step, one 128-column block
 * per lane, 8 KB of consecutive HBM bytes per step), then the n_o up rows. Each lane writes its
 * block's scaled double term to LDS; at the end lane r < 2*n_o adds the terms of buffered row
 * r in block order (the reference's sequential double sum), and lane r < n_o pairs gate row
 * r with up row n_o + r for the SwiGLU. n_o = G53GuShape<NBLK>::NO. Grid:
 * (ceil(nslots * I / n_o / 4), T), 256 threads. */

/* Agent-scope relaxed accesses: coherent across the XCDs' L2 caches (the compiler emits the
 * sc1 cache policy) without the L2 writeback / invalidate of a release / acquire fence. Used
 * for the few values one workgroup hands to another inside a kernel. */
__device__ __forceinline__ void g53_st_agent(float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float g53_ld_agent(const float *p)
{
    return __hip_atomic_load((float *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int g53_ld_agent_i(const int *p)
{
    return __hip_atomic_load((int *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* ----------------------------------------------------------------- router ---- */
/* Dot products in double. Every product of two floats is exact in double, so the only
 * rounding is in the additions; the reference adds sequentially, this adds per lane and
 * then across the wave. The double sums agree whenever the additions are exact (always
 * for bf16-valued router and input rows of ordinary range) and otherwise differ in the last
 * double bits, which changes the float score only if it lies within that distance of a
 * float rounding boundary. */
__device__ __forceinline__ float g53_router_dot(const void *gate, int dt, int e, int E, const float *x, int lane)
{
    double acc = 0.0;
    if (dt == 1 && E % 512 == 0) {
        /* bf16 rows: each lane takes E/64 consecutive weights, read 16 bytes at a time */
        const int per = E / 64;
        const uint16_t *row = (const uint16_t *)gate + (size_t)e * E + lane * per;
        const float *xl = x + lane * per;
        for (int i = 0; i < per; i += 8) {
            const uint4 q = *(const uint4 *)(row + i);
            const float4 x0 = *(const float4 *)(xl + i), x1 = *(const float4 *)(xl + i + 4);
            const uint32_t d[4] = {q.x, q.y, q.z, q.w};
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                acc += (double)g53_bitsf(d[k] << 16) * (double)xv[2 * k];
                acc += (double)g53_bitsf(d[k] & 0xffff0000u) * (double)xv[2 * k + 1];
            }
        }
    } else if (dt == 1) {
        const uint16_t *row = (const uint16_t *)gate + (size_t)e * E;
        for (int i = lane; i < E; i += 64)
            acc += (double)g53_bitsf((uint32_t)row[i] << 16) * (double)x[i];
    } else {
        const float *row = (const float *)gate + (size_t)e * E;
        for (int i = lane; i < E; i += 64) acc += (double)row[i] * (double)x[i];
    }
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    return (float)acc;
}



/* Loads of values another workgroup wrote in this kernel: a buffer load with the sc1 cache
 * policy (coherent across the XCDs), 16 bytes per lane. base must stay valid for the offset. */
__device__ __forceinline__ float4 g53_ld4_agent(const float *base, int byte_off)
{
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0x7fffffff,
                                                                       0x00020000);
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16));
}

/* Total order of floats as unsigned keys (larger float -> larger key; +0 and -0 equal). */
__device__ __forceinline__ uint32_t g53_fkey(float f)
{
    if (f == 0.0f) f = 0.0f;
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* The maximum (or minimum) of v over the wave, in every lane, without leaving the vector
 * unit: four DPP steps within each row of 16 lanes (lane xor 1, xor 2, the half-row mirror,
 * the row mirror), then the gfx950 row-pair and half-wave swaps. The whole wave must be
 * active. */
template <bool MAX>
__device__ __forceinline__ uint32_t g53_wall(uint32_t v)
{
    auto op = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xf, 0xf, true));   /* quad_perm 1,0,3,2 */
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xf, 0xf, true));   /* quad_perm 2,3,0,1 */
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, true));  /* row_half_mirror */
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xf, 0xf, true));  /* row_mirror */
    const auto p16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = op(p16[0], p16[1]);
    const auto p32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return op(p32[0], p32[1]);
}

#ifndef G53_SEL_PER_LANE
#define G53_SEL_PER_LANE 16   /* up to 1024 experts per wave */
#endif
/* route_topn (src/core/glm53f_ops.c:1021-1042): the scan starts from expert 0, so a NaN at
 * index 0 wins the round (the taken expert is then -inf) and NaN elsewhere is skipped. */
__device__ __forceinline__ void g53_topn_token(int t, int lane, int *__restrict__ idx, int n,
                                               const float *__restrict__ choice, int NE,
                                               const float *__restrict__ score, float *__restrict__ score_out)
{
    choice += (size_t)t * NE;
    idx += (size_t)t * n;
    float c[G53_SEL_PER_LANE];
    for (int k = 0; k < G53_SEL_PER_LANE; k++) {
        const int e = lane + 64 * k;
        c[k] = e < NE ? choice[e] : NAN;
    }
    /* a round: each lane's first strictly greater (its lowest expert among equal values), then
     * the wave's largest as a total-order key (+0 and -0 equal, 0 for no candidate) and the
     * lowest expert holding it, both reduced in every lane (the whole wave runs this) */
    for (int j = 0; j < n; j++) {
        int best;
        /* expert 0's value: a NaN there wins the round (and is -inf after it) */
        if (__builtin_isnan(__uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(c[0]))))) {
            best = 0;
        } else {
            float bv = -INFINITY;
            int bi = -1;
            for (int k = 0; k < G53_SEL_PER_LANE; k++) {
                const int e = lane + 64 * k;
                if (e < NE && c[k] == c[k] && (bi < 0 || c[k] > bv)) { bv = c[k]; bi = e; }
            }
            const uint32_t kb = bi < 0 ? 0u : g53_fkey(bv);
            const uint32_t m = g53_wall<true>(kb);
            const uint32_t lo = g53_wall<false>(kb == m && m != 0u ? (uint32_t)bi : 0xffffffffu);
            best = lo == 0xffffffffu ? 0 : (int)lo;
        }
        for (int k = 0; k < G53_SEL_PER_LANE; k++)
            if (lane + 64 * k == best) c[k] = -INFINITY;
        if (lane == 0) {
            idx[j] = best;
            if (score_out) score_out[(size_t)t * n + j] = score[(size_t)t * NE + best];
        }
    }
}

#endif /* G53H_GEMV_H */
