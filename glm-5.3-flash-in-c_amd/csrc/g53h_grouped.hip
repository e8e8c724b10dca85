/* g53h_grouped.hip - batched decode and prefill of the routed-expert MoE layer on gfx950:
 * token-sorted grouped GEMMs on the CDNA4 FP8 matrix cores.
 *
 * The reference runs a chunk of tokens expert by expert (src/core/glm53f_ops.c:1144-1342,
 * moe_chunk): route every token, gather the tokens of each chosen expert, apply gate/up,
 * the clamped SwiGLU and down to that group (matmul_f8_batch, :376-444), then combine each
 * token's slots in double in top-k order and add the shared expert (:1329-1340). This file
 * does the same with every expert's weights read from HBM once per call:
 *
 *   1. router             the exact router kernels of g53h_ops.hip (top-k bit-exact).
 *   2. k_grp_plan         counting sort of the (token, slot) pairs by expert, stable in token
 *                         order; segment e holds expert e's tokens, segment NE the shared
 *                         expert's (every token); a tile is <= 64 consecutive positions of one
 *                         segment.
 *   3. k_grp_xq           each token's activations as NPX E4M3 planes with a power-of-two
 *                         token scale: x = 2^-k (q0 + q1 / 16 + q2 / 256 ...). For bf16-valued
 *                         inputs two planes hold x exactly (8 significant bits = 4 + 4).
 *   4. k_grp_gateup       per (tile, 128-row block): gate and up rows of the expert times the
 *                         tile's tokens on v_mfma_scale_f32_32x32x64_f8f6f4, one 128x128 scale
 *                         block per step, the block scale applied to each block's fp32 sum;
 *                         SwiGLU in the epilogue; the activation leaves as NPA E4M3 planes with
 *                         a fixed power-of-two scale (|act| <= max(limit, 0.28) * limit).
 *   5. k_grp_down         per (tile, 256-row block): down rows times the activation planes;
 *                         contributions to contrib[position][hidden] (zeros for an absent
 *                         expert, the reference's drop path).
 *   6. k_grp_combine      out[t] = (float)(sum_j (double)w[t][j] * contrib[pos(t, j)]) in slot
 *                         order, then + shared contribution (float), as :1329-1340.
 *
 * Arithmetic: E4M3 x E4M3 products are exact in fp32; the matrix core sums them in fp32 in
 * its own order. So results differ from the reference's (fp32 FMA lanes, double block sums)
 * by fp32 summation order and by the activation planes' rounding, inside the tolerance the
 * path is held to (2e-3 relative + 1e-2 absolute per output). Routing is bit-exact.
 *
 * Operand layout of the 32x32x64 FP8 matrix instruction (one wave): lane l supplies row
 * l % 32 of A and column l % 32 of B, 32 K-bytes each, from K group l / 32; both operands use
 * the same K assignment, so any fixed map of K bytes to (group, byte) gives the same dot
 * product. Here group g of step s covers bytes g*64 + s*32 .. +32 of a 128-byte scale block,
 * so a lane reads 64 consecutive bytes of its weight row per block. Result: lane l, register
 * r holds C[8*(r/4) + 4*(l/32) + r%4][l % 32].
 *
 * Octet-tiled layers (G53H_MAT_TILED, the HBM cache's slots): a row's 128 bytes of a block are
 * the tiled unit's row, whose byte b holds column sigma(b / 16) + 8 (b % 16) of the block
 * (include/g53h.h). The activation planes are then written in that same order within every
 * 128-column block, so weight byte b meets activation byte b as before, and a wave's 32 rows of
 * a block are four whole 1 KB units instead of 32 rows 4 KB apart.
 */
#include <hip/hip_runtime.h>
#include <math.h>

#include "g53h.h"
#include "g53h_core.h"
#include "g53h_kern.h"
#include "g53h_runtime.h"

typedef int g53_v8i __attribute__((ext_vector_type(8)));
typedef float g53_v16f __attribute__((ext_vector_type(16)));
typedef int g53_v4i __attribute__((ext_vector_type(4)));
/* global-memory views, so loads are global_load (vector memory only), not flat */
typedef __attribute__((address_space(1))) const g53_v8i g53_gv8i;
typedef __attribute__((address_space(1))) const g53_v4i g53_gv4i;
typedef __attribute__((address_space(1))) const float g53_gflt;

#define G53_GRP_NT    128     /* positions per tile                                        */
#define G53_GRP_NH    (G53_GRP_NT / 32)   /* 32-position halves of a tile (matrix-core columns) */
#define G53_GRP_XST   144     /* LDS bytes per token row of a 128-byte slice (16 B padding) */
#define G53_GRP_MAXT  2048    /* tokens per planning pass                                   */
#define G53_GRP_NPX   2       /* E4M3 planes of the input activations                       */
#define G53_GRP_NPA   2       /* E4M3 planes of the SwiGLU activations                      */
#define G53_GRP_MASKS 12288   /* LDS 64-token masks of the planner (chunks x experts)       */
#define G53_GRP_NW    8       /* waves of a GEMM workgroup                                   */
#ifndef G53_GRP_WPC
#define G53_GRP_WPC   1       /* GEMM workgroups resident per CU                             */
#endif
#ifndef G53_GRP_PERS
#define G53_GRP_PERS  1       /* workgroups per CU in the grid: each loops over its items  */
#endif
#ifndef G53_GRP_RS
#define G53_GRP_RS    2       /* weight blocks in a lane's ring                              */
#endif
#ifndef G53_GRP_LXS
#define G53_GRP_LXS   2       /* activation slices in a thread's ring                        */
#endif
#ifndef G53_GRP_NS
#define G53_GRP_NS    2       /* activation slices in the workgroup's LDS ring               */
#endif

/* error flags (meta[1]) */
#define G53_GRP_EIDX  1       /* a routed index outside [0, n_experts)                      */
#define G53_GRP_EDESC 8       /* an expert descriptor without the expected 128x128 layout   */
#define G53_GRP_ESPIN 2       /* a wait on the slice ring timed out                          */

/* ------------------------------------------------------------------ planning ---- */
/* meta[]: [0] tiles, [1] error flags, [2..17] the GEMMs' item counters, then the first item of
 * each XCD's range (9 entries: XCD x takes items [b[x], b[x+1])) for gate/up and for down */
#define G53_GRP_BGU   18
#define G53_GRP_BDN   27

/* Estimated cost of one row of a segment's items (one item per tile) with n positions, in
 * tenths of the time of a tile of at most 64 positions. Measured item times at 1, 2, 3 and 4
 * 32-position halves were 47, 51, 63 and 70 us: up to two halves the weight stream alone sets
 * the time, beyond that the matrix work adds about a third per half. */
__device__ __forceinline__ int g53_grp_tile_cost(int n)
{
    const int h = (n + 31) / 32;
    return h <= 2 ? 10 : 10 + 3 * (h - 2) - (h == 4 ? 1 : 0);
}
__device__ __forceinline__ int g53_grp_seg_cost(int n)
{
    const int full = n / G53_GRP_NT, rem = n % G53_GRP_NT;
    return full * g53_grp_tile_cost(G53_GRP_NT) + (rem ? g53_grp_tile_cost(rem) : 0);
}

/* Counting sort of the T*K (token, slot) pairs by expert, stable in token order. For each
 * chunk c of 64 tokens and expert e, mask[c][e] has bit t%64 set when token t chose e; the
 * position of (t, e) is off[e] + (tokens of e in earlier chunks) + popcount(mask bits below
 * t). One workgroup of 1024 threads; dynamic LDS sized by the host. */
__global__ void __launch_bounds__(1024)
k_grp_plan(const int *__restrict__ idx, int T, int K, int NE, int has_sh, int *__restrict__ tok_of,
           int *__restrict__ pos_of, int4 *__restrict__ tiles, int *__restrict__ meta, int mb_gu, int mb_dn)
{
    extern __shared__ __attribute__((aligned(16))) uint64_t pl_lds[];
    const int nch = (T + 63) >> 6, nm = nch * NE, tid = threadIdx.x;
    uint64_t *mask = pl_lds;
    int *pre = (int *)(mask + nm);                 /* [nch][NE]                              */
    int *off = pre + nm;                           /* [NE + 2]: segment offsets              */
    int *tb = off + NE + 2;                        /* [NE + 2]: first tile of each segment   */
    int *pc = tb + NE + 2;                         /* [NE + 2]: cost of the segments before  */
    const int nseg = NE + (has_sh ? 1 : 0);
    for (int i = tid; i < nm; i += 1024) mask[i] = 0;
    __syncthreads();
    int bad = 0;
    for (int f = tid; f < T * K; f += 1024) {
        const int t = f / K, e = idx[f];
        if (e < 0 || e >= NE) { bad = 1; continue; }
        atomicOr((unsigned long long *)&mask[(t >> 6) * NE + e], 1ull << (t & 63));
    }
    if (bad) atomicOr(&meta[1], G53_GRP_EIDX);
    __syncthreads();
    /* per expert: tokens in earlier chunks, and the count (into off[] for the scan below) */
    for (int e = tid; e < NE; e += 1024) {
        int run = 0;
        for (int c = 0; c < nch; c++) {
            pre[c * NE + e] = run;
            run += __popcll(mask[c * NE + e]);
        }
        off[e] = run;
    }
    if (tid == 0) off[NE] = has_sh ? T : 0;
    __syncthreads();
    /* exclusive scans of counts and tile counts by the first wave, 64 segments per round */
    if (tid < 64) {
        int cp = 0, ct = 0, cc = 0;
        for (int b = 0; b < nseg; b += 64) {
            const int s = b + tid;
            const int n = s < nseg ? off[s] : 0;
            const int c = g53_grp_seg_cost(n);
            int ip = n, it = (n + G53_GRP_NT - 1) / G53_GRP_NT, ic = c;
            for (int d = 1; d < 64; d <<= 1) {
                const int up = __shfl_up(ip, d), ut = __shfl_up(it, d), uc = __shfl_up(ic, d);
                if (tid >= d) { ip += up; it += ut; ic += uc; }
            }
            if (s < nseg) {
                off[s] = cp + ip - n;
                tb[s] = ct + it - (n + G53_GRP_NT - 1) / G53_GRP_NT;
                pc[s] = cc + ic - c;
            }
            cp += __shfl(ip, 63);
            ct += __shfl(it, 63);
            cc += __shfl(ic, 63);
        }
        if (tid == 0) { off[nseg] = cp; tb[nseg] = ct; pc[nseg] = cc; meta[0] = ct; }
        if (tid < 16) meta[2 + tid] = 0;         /* the GEMMs' item counters */
    }
    __syncthreads();
    /* each XCD's item range, of equal estimated cost: lanes 0-8 for gate/up, 16-24 for down */
    if (tid < 32 && (tid & 15) <= 8) {
        const int x = tid & 15, MB = tid < 16 ? mb_gu : mb_dn;
        int item;
        if (x == 0) item = 0;
        else if (x == 8) item = tb[nseg] * MB;
        else {
            const long long tau = (long long)pc[nseg] * x / 8;   /* target, in units of one row of items */
            int lo = 0, hi = nseg;                                /* the last segment with pc <= tau */
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (pc[mid] <= tau) lo = mid; else hi = mid - 1;
            }
            item = tb[lo] * MB;
            if (lo < nseg) {
                const int rc = pc[lo + 1] - pc[lo], nts = tb[lo + 1] - tb[lo];
                const long long j = rc > 0 ? ((tau - pc[lo]) * MB) / rc : 0;   /* whole rows of items */
                item += (int)(j < MB ? j : MB) * nts;
            }
        }
        meta[(tid < 16 ? G53_GRP_BGU : G53_GRP_BDN) + x] = item;
    }
    __syncthreads();
    const int ps = K + 1;
    for (int f = tid; f < T * K; f += 1024) {
        const int t = f / K, j = f % K, e = idx[f];
        if (e < 0 || e >= NE) { pos_of[t * ps + j] = -1; continue; }
        const int c = t >> 6;
        const uint64_t m = mask[c * NE + e];
        const int pos = off[e] + pre[c * NE + e] + __popcll(m & ((1ull << (t & 63)) - 1ull));
        pos_of[t * ps + j] = pos;
        tok_of[pos] = t;
    }
    if (has_sh)
        for (int t = tid; t < T; t += 1024) {
            const int pos = off[NE] + t;
            pos_of[t * ps + K] = pos;
            tok_of[pos] = t;
        }
    for (int s = tid; s < nseg; s += 1024) {
        const int n = off[s + 1] - off[s];
        const int nt = (n + G53_GRP_NT - 1) / G53_GRP_NT;
        for (int i = 0; i < nt; i++) {
            const int m = n - i * G53_GRP_NT;
            tiles[tb[s] + i] = make_int4(s, off[s] + i * G53_GRP_NT, m < G53_GRP_NT ? m : G53_GRP_NT, tb[s] | nt << 16);
        }
    }
}

/* ------------------------------------------------------------ E4M3 planes ---- */
/* Four values v[0..3] (already scaled into E4M3 range) as NP planes of packed E4M3 bytes:
 * plane p holds round(r_p * 16^p), r_0 = v, r_{p+1} = r_p - plane p's value / 16^p. */
template <int NP>
__device__ __forceinline__ void g53_split_planes(const float (&v)[4], uint32_t (&out)[NP])
{
    float r[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
    for (int p = 0; p < NP; p++) {
        int w = __builtin_amdgcn_cvt_pk_fp8_f32(r[0], r[1], 0, false);
        w = __builtin_amdgcn_cvt_pk_fp8_f32(r[2], r[3], w, true);
        out[p] = (uint32_t)w;
        if (p + 1 < NP) {
            r[0] = (r[0] - __builtin_amdgcn_cvt_f32_fp8(w, 0)) * 16.0f;
            r[1] = (r[1] - __builtin_amdgcn_cvt_f32_fp8(w, 1)) * 16.0f;
            r[2] = (r[2] - __builtin_amdgcn_cvt_f32_fp8(w, 2)) * 16.0f;
            r[3] = (r[3] - __builtin_amdgcn_cvt_f32_fp8(w, 3)) * 16.0f;
        }
    }
}

/* Token t's row of x as NPX planes xq[p][t][E] with scale 2^k, k = 8 - exponent(absmax), so
 * every |x| * 2^k < 256; xinv[t] = 2^-k. Grid T, 256 threads, E a multiple of 16. */
/* Byte position of column c of a 128-column block in the octet-tiled order: run sigma(c % 8)
 * (sigma is its own inverse), element c / 8 of the run. */
__device__ __forceinline__ int g53_grp_tpos(int c)
{
    const int a = c & 7;
    return 16 * (((a & 1) << 2) | (a & 2) | (a >> 2)) + (c >> 3);
}

/* Four consecutive E4M3 codes (one word, column c0 .. c0 + 3 of a row) stored at dst: as they
 * are, or (tiled) each at its octet-tiled position within its 128-column block. */
__device__ __forceinline__ void g53_grp_st4(uint8_t *row, int c0, uint32_t q, int tiled)
{
    if (!tiled) {
        *(uint32_t *)(row + c0) = q;
        return;
    }
    uint8_t *blk = row + (c0 & ~127);
#pragma unroll
    for (int k = 0; k < 4; k++) blk[g53_grp_tpos((c0 + k) & 127)] = (uint8_t)(q >> (8 * k));
}

template <int NP>
__global__ void __launch_bounds__(256)
k_grp_xq(const float *__restrict__ x, int E, int T, uint8_t *__restrict__ xq, float *__restrict__ xinv, int tiled)
{
    __shared__ float red[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float *xr = x + (size_t)t * E;
    float m = 0.0f;
    for (int i = tid * 4; i < E; i += 1024) {
        const float4 v = *(const float4 *)(xr + i);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int ex = 0;
    if (m > 0.0f && m <= 3.0e38f) (void)frexpf(m, &ex);          /* m < 2^ex */
    const int k = 8 - ex;
    const float sc = ldexpf(1.0f, k);
    if (tid == 0) xinv[t] = ldexpf(1.0f, -k);
    for (int i = tid * 4; i < E; i += 1024) {
        const float4 v = *(const float4 *)(xr + i);
        const float s[4] = {v.x * sc, v.y * sc, v.z * sc, v.w * sc};
        uint32_t q[NP];
        g53_split_planes<NP>(s, q);
#pragma unroll
        for (int p = 0; p < NP; p++) g53_grp_st4(xq + ((size_t)p * T + t) * E, i, q[p], tiled);
    }
}

/* ------------------------------------------------------------- grouped GEMM ---- */
/* A workgroup = NW waves; wave w owns 32 rows of A (rows chosen by the caller) and both
 * 32-position halves of a 64-position tile. Two workgroups share a CU, so one's matrix work
 * overlaps the other's waits at its per-block barrier. The K loop walks 128-byte scale blocks.
 * Per block kb a thread issues, in this order, its 16-byte pieces of the activation slice
 * kb + LX (a ring of LX register slots) and its lane's 64 weight bytes of block kb + R - 1 (a
 * ring of R slots), runs block kb on the matrix cores from LDS slice kb, then stores slice
 * kb + 1 to the other LDS buffer. Loads complete in issue order, so that store waits for the
 * weights up to block kb + LX - 1 only, issued LX + 1 blocks earlier. */
template <int NP, int NH>
__device__ __forceinline__ void g53_grp_block(g53_v16f (&acc)[G53_GRP_NH], const g53_v8i &w0, const g53_v8i &w1,
                                              const uint8_t *xb, int c0b, int c1b)
{
    const float c0 = __int_as_float(c0b), c1 = __int_as_float(c1b);
#pragma unroll
    for (int h = 0; h < NH; h++) {
        g53_v16f b = {};
#pragma unroll
        for (int p = 0; p < NP; p++) {
#pragma unroll
            for (int s = 0; s < 2; s++) {
                const g53_v8i x = *(const g53_v8i *)(xb + p * G53_GRP_NT * G53_GRP_XST + h * 32 * G53_GRP_XST + s * 32);
                b = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(s ? w1 : w0, x, b, 0, 0, 0, 127, 0, 127 - 4 * p);
            }
        }
#pragma unroll
        for (int r = 0; r < 16; r++) acc[h][r] = fmaf(b[r], r < 8 ? c0 : c1, acc[h][r]);
        /* pin the half's arithmetic here: the compiler would otherwise sink the pure matrix
         * arithmetic past the ring waits to the loop's end and keep every block's operands live */
        asm volatile("" : "+v"(acc[h]));
    }
}

#ifdef G53_GRP_KTRACE
__device__ uint64_t *g53_ktrace;     /* diagnostic builds only: per-block timestamps */
extern "C" int g53h_set_grouped_ktrace(void *p)
{
    return hipMemcpyToSymbol(HIP_SYMBOL(g53_ktrace), &p, sizeof p) == hipSuccess ? 0 : -1;
}
#endif

/* LDS counters of the slice ring: relaxed workgroup-scope atomics (a wave's LDS operations
 * execute in order, so a count added after a wave's slice stores is seen after them), and a
 * bounded sleep-poll that reports a timeout instead of hanging. */
#define G53_CBAR() asm volatile("" ::: "memory")
__device__ __forceinline__ void g53_grp_lds_add(int *p, int v)
{
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ int g53_grp_wait(int *p, int want)
{
    int spins = 0;
    while (__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < want) {
        if (++spins > (1 << 22)) return 1;
        __builtin_amdgcn_s_sleep(1);
    }
    G53_CBAR();
    return 0;
}

/* The activation slice loader of a workgroup of NW waves: a slice is G53_GRP_NT positions x
 * 128 bytes x NP planes, 16-byte pieces; thread t takes piece t % 8 of positions
 * t / 8 + j * 8 * NW. */
template <int NW>
struct G53GrpLd {
    static constexpr int RPT = G53_GRP_NT * 8 / (64 * NW);   /* positions per thread    */
    const uint8_t *src[RPT];                           /* source rows (+ 16 * piece)     */
    int dst[RPT];                                      /* LDS offsets in a slice         */
};

/* acc[h][r] += scale_r * (A_rows x B_tile-half-h), h < NH, over NKB blocks of 128 bytes.
 *   arow    this lane's weight row + (l / 32) * 64 (block 0), kst bytes to the next block
 *           (128 row-major, 1024 octet-tiled)
 *   s0, s1  scale rows for C registers 0-7 and 8-15 (one float per block)
 *   ld      this thread's slice loader; plane p of a source row at + p * xps
 *   NH      32-position halves the tile has (positions beyond the tile's count are padding) */
template <int NW, int NP, int NKB, int NH>
__device__ __forceinline__ void g53_grp_kloop(g53_v16f (&acc)[G53_GRP_NH], const uint8_t *arow, int kst, const float *s0,
                                              const float *s1, const G53GrpLd<NW> &ld, size_t xps, uint8_t *xs,
                                              int *flags, int &spin_err, int lane)
{
    constexpr int SL = NP * G53_GRP_NT * G53_GRP_XST;           /* one slice in LDS        */
    constexpr int PL = G53_GRP_NT * G53_GRP_XST;                /* one plane of a slice    */
    /* only the rows the NH halves read are loaded: positions >= 32 * NH are never used */
    constexpr int RPT0 = G53GrpLd<NW>::RPT, RPN = (NH * 32 + 8 * NW - 1) / (8 * NW);
    constexpr int RPT = RPN < RPT0 ? RPN : RPT0;
    constexpr int LX = G53_GRP_LXS;                             /* slice slots             */
    constexpr int R0 = G53_GRP_RS;                              /* weight slots            */
    constexpr int R = NKB < R0 ? NKB : R0;
    constexpr int NS = G53_GRP_NS;                              /* LDS slice slots         */
    static_assert(NKB % R == 0 && R % LX == 0 && R % NS == 0, "ring sizes");
    int *ready = flags, *freed = flags + NS;
    static_assert(NKB <= 64, "one scale per lane");
    static_assert(NP == 2 || NP == 3, "two or three planes");
    const uint8_t *xrd = xs + (lane >> 5) * 64 + (lane & 31) * G53_GRP_XST;
    /* the block scales of the wave's rows, lane k holding block k's (loaded once, before any
     * weight load, so no later wait on them waits for weights) */
    const float sv0 = lane < NKB ? ((g53_gflt *)s0)[lane] : 0.0f, sv1 = lane < NKB ? ((g53_gflt *)s1)[lane] : 0.0f;
    g53_v8i a[R][2];
    g53_v4i xr[LX][RPT][3];
    typedef const __attribute__((address_space(1))) uint8_t *gptr;
    const gptr ag = (gptr)arow;
    gptr xg[RPT];
#pragma unroll
    for (int j = 0; j < RPT; j++) xg[j] = (gptr)ld.src[j];
#define G53_LDA(sl, k) do { a[sl][0] = *(g53_gv8i *)(ag + (size_t)(k) * kst); a[sl][1] = *(g53_gv8i *)(ag + (size_t)(k) * kst + 32); } while (0)
#define G53_LDX(sl, k) do { _Pragma("unroll") for (int j = 0; j < RPT; j++) {                                  \
                                xr[sl][j][0] = *(g53_gv4i *)(xg[j] + (k) * 128);                               \
                                xr[sl][j][1] = *(g53_gv4i *)(xg[j] + xps + (k) * 128);                         \
                                if (NP == 3) xr[sl][j][2] = *(g53_gv4i *)(xg[j] + 2 * xps + (k) * 128); } } while (0)
#define G53_STX(sl, buf) do { _Pragma("unroll") for (int j = 0; j < RPT; j++) {                                \
                                  uint8_t *d_ = xs + (buf) * SL + ld.dst[j];                                   \
                                  *(g53_v4i *)d_ = xr[sl][j][0]; *(g53_v4i *)(d_ + PL) = xr[sl][j][1];         \
                                  if (NP == 3) *(g53_v4i *)(d_ + 2 * PL) = xr[sl][j][2]; } } while (0)
    /* prologue: slices 0 .. LX-1 (slice 0 to LDS), then the weights of blocks 0 .. R-2 */
#pragma unroll
    for (int k = 0; k < LX; k++) G53_LDX(k, k < NKB ? k : NKB - 1);
#pragma unroll
    for (int k = 0; k < R - 1; k++) G53_LDA(k, k);
    G53_STX(0, 0);
    G53_CBAR();
    if (lane == 0) g53_grp_lds_add(&ready[0], 1);
    /* Block kb: issue slice kb+LX and weights kb+R-1; store slice kb+1 into its slot once every
     * wave has finished the block that slot held (freed), and count it ready; wait until every
     * wave has stored slice kb (ready), multiply, count it freed. No workgroup barrier: waves
     * drift up to NS-1 blocks apart. Loads past the end re-read the last block. */
#pragma nounroll
    for (int kb0 = 0; kb0 < NKB; kb0 += R) {
#pragma unroll
        for (int u = 0; u < R; u++) {
            const int kb = kb0 + u;
            const int kx = kb + LX < NKB ? kb + LX : NKB - 1;
            const int ka = kb + R - 1 < NKB ? kb + R - 1 : NKB - 1;
#ifdef G53_GRP_KTRACE
            uint64_t kt0 = __builtin_amdgcn_s_memrealtime(), kt1 = 0, kt2 = 0;
#endif
            G53_LDX(u % LX, kx);
            G53_LDA((u + R - 1) % R, ka);
            if (kb + 1 < NKB) {
                const int sn = (u + 1) % NS;
                spin_err |= g53_grp_wait(&freed[sn], NW * ((kb + 1) / NS));
                G53_STX((u + 1) % LX, sn);
                G53_CBAR();
                if (lane == 0) g53_grp_lds_add(&ready[sn], 1);
            }
#ifdef G53_GRP_KTRACE
            kt1 = __builtin_amdgcn_s_memrealtime();
#endif
            spin_err |= g53_grp_wait(&ready[u % NS], NW * (kb / NS + 1));
#ifdef G53_GRP_KTRACE
            kt2 = __builtin_amdgcn_s_memrealtime();
#endif
            g53_grp_block<NP, NH>(acc, a[u][0], a[u][1], xrd + (u % NS) * SL,
                                   __builtin_amdgcn_readlane(__float_as_int(sv0), kb),
                                   __builtin_amdgcn_readlane(__float_as_int(sv1), kb));
            G53_CBAR();
            if (lane == 0) g53_grp_lds_add(&freed[u % NS], 1);
#ifdef G53_GRP_KTRACE
            if (g53_ktrace && lane == 0 && NKB == 32) {   /* the gate/up kernel */
                uint64_t *o = g53_ktrace + (((size_t)blockIdx.x * NW + (threadIdx.x >> 6)) * 32 + kb) * 4;
                o[0] = kt0; o[1] = kt1; o[2] = kt2; o[3] = __builtin_amdgcn_s_memrealtime();
            }
#endif
            __builtin_amdgcn_sched_barrier(0);   /* keep the blocks in program order */
        }
    }
#undef G53_LDA
#undef G53_LDX
#undef G53_STX
}

/* A descriptor with the layout the grouped kernels assume (octet-tiled iff the pass is). */
__device__ __forceinline__ bool g53_grp_desc_ok(const G53hExpert &x, int E, int I, int tiled)
{
    const int want = tiled ? G53H_MAT_TILED : 0;
    return !((x.gate.flags | x.up.flags | x.down.flags) & G53H_MAT_I4) &&
           (x.gate.flags & G53H_MAT_TILED) == want && (x.up.flags & G53H_MAT_TILED) == want &&
           (x.down.flags & G53H_MAT_TILED) == want &&
           x.gate.br == 128 && x.gate.bc == 128 && x.gate.rows == I && x.gate.cols == E &&
           x.up.br == 128 && x.up.bc == 128 && x.up.rows == I && x.up.cols == E &&
           x.down.br == 128 && x.down.bc == 128 && x.down.rows == E && x.down.cols == I &&
           x.gate.scols >= E / 128 && x.up.scols >= E / 128 && x.down.scols >= I / 128;
}

struct G53GrpArgs {
    const G53hExpert *experts;     /* [NE]                                               */
    const G53hExpert *shared;      /* or NULL                                            */
    const int4 *tiles;             /* {segment, first position, count, first tile of the
                                      segment | tiles of the segment << 16}                */
    const int *meta;               /* [0] tile count, [1] error flags                    */
    int *meta_w;
    const int *tok_of;             /* position -> token                                  */
    const uint8_t *xq;             /* [NPX][T][E]                                        */
    const float *xinv;             /* [T]                                                */
    uint8_t *aq;                   /* [NPA][P][I]                                        */
    float *contrib;                /* [P][E]                                             */
    int T, P, E, I, NE;
    float limit, aq_scale, aq_inv;
    int tiled;                     /* 1: experts octet-tiled, planes in the tiled column order */
    int partial;                   /* 1: experts without weights are outside this batch and
                                      left alone, unless marked dropped (gate.flags & G53H_MAT_DROPPED)    */
    int *ctr;                      /* [16] item counters: 0-7 gate/up, 8-15 down; each
                                      kernel starts with its own at zero and clears the
                                      other kernel's                                      */
    uint64_t *trace;               /* optional: [grid][8] timestamps of each workgroup    */
};

/* Diagnostics: 100 MHz timestamps of an item's phases into a.trace[item * 8 + k] when it is set
 * (gti: the item's number). */
#define G53_GTRACE(k, v) do { if (a.trace && threadIdx.x == 0) a.trace[(size_t)gti * 32 + (k)] = (v); } while (0)
#define G53_GTRACE_W(k, v) do { if (a.trace && (threadIdx.x & 63) == 0) a.trace[(size_t)gti * 32 + (k)] = (v); } while (0)

/* Item loc of the workgroup's group: the dispatcher deals workgroups round-robin over the 8
 * XCDs, so the workgroups of XCD x (blockIdx.x % 8 == x) share the items blo .. bhi - 1 (a
 * range of equal estimated cost, from the planner), which they claim in order from the
 * group's counter. Items are numbered segment by segment, and inside a segment row block by
 * row block, all tiles of a block in a row: the tiles of one expert that re-read the same
 * weight rows run next to each other on one XCD and find them in its L2. Returns false past
 * the group's last item. */
__device__ __forceinline__ bool g53_grp_item(const int4 *tiles, int blo, int bhi, int MB, int loc, int4 &tl, int &mb)
{
    const int item = blo + loc;
    if (item >= bhi) return false;
    const int w = tiles[item / MB].w;                    /* a tile of the item's segment */
    const int ts0 = w & 0xffff, nts = w >> 16;
    const int q = item - ts0 * MB;
    mb = q / nts;
    tl = tiles[ts0 + q % nts];
    return true;
}

/* Claim the group's next item (a relaxed device-scope counter, one claim per item, issued an
 * item ahead so that its latency hides behind the current item). */
__device__ __forceinline__ int g53_grp_claim(int *ctr)
{
    return __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Gate/up + SwiGLU for (tile, block mb of 16*NW intermediate rows). Wave w: A rows 0-15 = gate
 * rows mb*16*NW + w*16 + 0..15, rows 16-31 = the up rows of the same indices, so C registers r
 * and r + 8 of a lane are gate and up of one intermediate row and one position. */
/* The clamped SwiGLU of src/core/glm53f_ops.c:486-494 (gate clamped from above, up both ways)
 * with the hardware exponential: the result is rounded to two E4M3 planes (about 8 significant
 * bits) right after, so the reference's expf to the last bit buys nothing here, and the exact
 * table method's LDS lookups queue behind the K loop's operand reads of the other waves (about
 * 3 us per 32 positions). Infinities and NaN follow the reference: sigmoid(-inf) = 0. */
__device__ __forceinline__ float g53_grp_swiglu(float g, float u, float limit)
{
    const float gi = g > limit ? limit : g;
    const float ui = u > limit ? limit : (u < -limit ? -limit : u);
    return gi * __frcp_rn(1.0f + __expf(-gi)) * ui;
}

template <int NW, int NKB>
__global__ void __launch_bounds__(64 * NW, G53_GRP_WPC) k_grp_gateup(G53GrpArgs a)
{
    __shared__ __attribute__((aligned(16))) uint8_t xs[G53_GRP_NS * G53_GRP_NPX * G53_GRP_NT * G53_GRP_XST];
    __shared__ __attribute__((aligned(16))) uint8_t ao[G53_GRP_NPA * G53_GRP_NT * 128];   /* the item's planes */
    __shared__ float xil[G53_GRP_NT];                    /* the tile's token scales          */
    __shared__ int flags[2 * G53_GRP_NS];
    __shared__ int claim[2];
    static_assert(16 * NW == 128, "an item is one 128-row scale block");
    int *ctr = a.ctr + (blockIdx.x & 7);
    if (threadIdx.x == 0) claim[0] = g53_grp_claim(ctr);
    if (blockIdx.x == 0 && threadIdx.x < 8) a.ctr[8 + threadIdx.x] = 0;   /* the down kernel's */
    const int blo = a.meta[G53_GRP_BGU + (blockIdx.x & 7)], bhi = a.meta[G53_GRP_BGU + (blockIdx.x & 7) + 1];
    for (int kk = 0;; kk++) {
        __syncthreads();                     /* claim[] written; the previous item is done with LDS */
        int4 tl;
        int mb;
        const uint64_t t_item = __builtin_amdgcn_s_memrealtime();
        if (!g53_grp_item(a.tiles, blo, bhi, a.I / (16 * NW), claim[kk & 1], tl, mb)) break;
        const int gti = blo + claim[kk & 1];
        G53_GTRACE(0, t_item);
        int nxt = 0;
        if (threadIdx.x == 0) nxt = g53_grp_claim(ctr);
        G53_GTRACE(4, (uint64_t)__smid() << 32 | (uint32_t)(tl.y << 8 | tl.z));
        G53_GTRACE(5, (uint64_t)blockIdx.x << 32 | (uint32_t)(tl.x << 8 | mb));
        const G53hExpert *ex = tl.x < a.NE ? &a.experts[tl.x] : a.shared;
        const bool usable = ex && ex->gate.w != nullptr && g53_grp_desc_ok(*ex, a.E, a.I, a.tiled);
        if (!usable) {                                       /* absent expert: down writes zeros */
            if (ex && ex->gate.w && threadIdx.x == 0) atomicOr(&a.meta_w[1], G53_GRP_EDESC);
            if (threadIdx.x == 0) claim[(kk + 1) & 1] = nxt;
            continue;
        }
        const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
        const int n = tl.z, pos0 = tl.y;
        G53GrpLd<NW> ld;
#pragma unroll
        for (int j = 0; j < G53GrpLd<NW>::RPT; j++) {
            const int lp = (tid >> 3) + j * 8 * NW, piece = tid & 7;
            ld.src[j] = a.xq + (size_t)a.tok_of[pos0 + (lp < n ? lp : 0)] * a.E + piece * 16;
            ld.dst[j] = lp * G53_GRP_XST + piece * 16;
        }
        const size_t xps = (size_t)a.T * a.E;
        /* this lane's weight row */
        const int i = lane & 31, g = lane >> 5;
        const int r0 = mb * 16 * NW + w * 16;                /* first intermediate row of the wave */
        const G53hMat &m = i < 16 ? ex->gate : ex->up;
        const int wr = r0 + (i & 15);
        const uint8_t *arow = a.tiled ? m.w + (size_t)(wr >> 3) * NKB * 1024 + (wr & 7) * 128 + g * 64
                                      : m.w + (size_t)wr * a.E + g * 64;
        const int kst = a.tiled ? 1024 : 128;
        const float *s0 = (const float *)ex->gate.s + (size_t)(r0 / 128) * ex->gate.scols;
        const float *s1 = (const float *)ex->up.s + (size_t)(r0 / 128) * ex->up.scols;
        g53_v16f acc[G53_GRP_NH] = {};
        /* the token scales of the tile's positions into LDS before the weights stream (read in
         * registers at the end, the compiler would load them there, behind the weights) */
        if (tid < n) xil[tid] = a.xinv[a.tok_of[pos0 + tid]];
        G53_GTRACE(1, __builtin_amdgcn_s_memrealtime());
        if (threadIdx.x < 2 * G53_GRP_NS) flags[threadIdx.x] = 0;
        if (threadIdx.x == 0) claim[(kk + 1) & 1] = nxt;
        __syncthreads();
        float xi[G53_GRP_NH];                                /* this lane's positions' scales */
#pragma unroll
        for (int h = 0; h < G53_GRP_NH; h++) xi[h] = xil[h * 32 + i];
        int spin_err = 0;
        switch ((n + 31) >> 5) {
        case 1: g53_grp_kloop<NW, G53_GRP_NPX, NKB, 1>(acc, arow, kst, s0, s1, ld, xps, xs, flags, spin_err, lane); break;
        case 2: g53_grp_kloop<NW, G53_GRP_NPX, NKB, 2>(acc, arow, kst, s0, s1, ld, xps, xs, flags, spin_err, lane); break;
        case 3: g53_grp_kloop<NW, G53_GRP_NPX, NKB, 3>(acc, arow, kst, s0, s1, ld, xps, xs, flags, spin_err, lane); break;
        default: g53_grp_kloop<NW, G53_GRP_NPX, NKB, 4>(acc, arow, kst, s0, s1, ld, xps, xs, flags, spin_err, lane); break;
        }
        if (spin_err && lane == 0) atomicOr(&a.meta_w[1], G53_GRP_ESPIN);
        G53_GTRACE(2, __builtin_amdgcn_s_memrealtime());
        G53_GTRACE_W(8 + w, __builtin_amdgcn_s_memrealtime());
        /* epilogue: SwiGLU; the activation planes of the item's 128 rows go to LDS in their final
         * byte order (the tiled order within the 128-column block when the pass is tiled), then
         * leave as whole 16-byte pieces: a lane's own bytes are scattered over 64 positions, and
         * storing them one by one from each lane costs the address unit about 3 us per 32
         * positions */
#pragma unroll
        for (int h = 0; h < G53_GRP_NH; h++) {
            const int j = h * 32 + i;
            if (j >= n) continue;
            uint32_t pk[2][G53_GRP_NPA];
#pragma unroll
            for (int q = 0; q < 2; q++) {
                float v[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int r = q * 4 + k;
                    v[k] = g53_grp_swiglu(acc[h][r] * xi[h], acc[h][r + 8] * xi[h], a.limit) * a.aq_scale;
                }
                g53_split_planes<G53_GRP_NPA>(v, pk[q]);
            }
            /* C register q * 4 + k holds local row w * 16 + q * 8 + g * 4 + k of the block */
#pragma unroll
            for (int p = 0; p < G53_GRP_NPA; p++) {
                uint8_t *d = ao + (p * G53_GRP_NT + j) * 128;
                if (a.tiled) {          /* rows of q = 0 and 1 are neighbouring bytes of one run */
#pragma unroll
                    for (int k = 0; k < 4; k++)
                        *(uint16_t *)(d + (g53_grp_tpos(g * 4 + k) & ~15) + 2 * w) =
                            (uint16_t)(((pk[0][p] >> (8 * k)) & 0xffu) | (((pk[1][p] >> (8 * k)) & 0xffu) << 8));
                } else {
                    *(uint32_t *)(d + w * 16 + g * 4) = pk[0][p];
                    *(uint32_t *)(d + w * 16 + 8 + g * 4) = pk[1][p];
                }
            }
        }
        __syncthreads();
        for (int c = tid; c < n * G53_GRP_NPA * 8; c += 64 * NW) {
            const int p = c / (n * 8), jq = c - p * n * 8, j = jq >> 3, piece = jq & 7;
            *(g53_v4i *)(a.aq + ((size_t)p * a.P + pos0 + j) * a.I + mb * 128 + piece * 16) =
                *(const g53_v4i *)(ao + (p * G53_GRP_NT + j) * 128 + piece * 16);
        }
        G53_GTRACE(3, __builtin_amdgcn_s_memrealtime());
        G53_GTRACE_W(16 + w, __builtin_amdgcn_s_memrealtime());
    }
}

/* Down for (tile, block mb of 32*NW rows): wave w owns rows mb*32*NW + w*32 + 0..31 of the down
 * matrix (inside one 128-row scale block), the tile's activation planes are the B operand. */
template <int NW, int NKB>
__global__ void __launch_bounds__(64 * NW, G53_GRP_WPC) k_grp_down(G53GrpArgs a)
{
    __shared__ __attribute__((aligned(16))) uint8_t xs[G53_GRP_NS * G53_GRP_NPA * G53_GRP_NT * G53_GRP_XST];
    __shared__ int flags[2 * G53_GRP_NS];
    __shared__ int claim[2];
    constexpr int MR = 32 * NW;
    int *ctr = a.ctr + 8 + (blockIdx.x & 7);
    if (threadIdx.x == 0) claim[0] = g53_grp_claim(ctr);
    if (blockIdx.x == 0 && threadIdx.x < 8) a.ctr[threadIdx.x] = 0;        /* the gate/up kernel's */
    const int blo = a.meta[G53_GRP_BDN + (blockIdx.x & 7)], bhi = a.meta[G53_GRP_BDN + (blockIdx.x & 7) + 1];
    for (int kk = 0;; kk++) {
        __syncthreads();                     /* claim[] written; the previous item is done with LDS */
        int4 tl;
        int mb;
        if (!g53_grp_item(a.tiles, blo, bhi, a.E / MR, claim[kk & 1], tl, mb)) break;
        int nxt = 0;
        if (threadIdx.x == 0) nxt = g53_grp_claim(ctr);
        const G53hExpert *ex = tl.x < a.NE ? &a.experts[tl.x] : a.shared;
        const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
        const int n = tl.z, pos0 = tl.y;
        const int i = lane & 31, g = lane >> 5;
        const bool present = ex && ex->gate.w != nullptr;
        if (!present && a.partial && !(ex && (ex->gate.flags & G53H_MAT_DROPPED))) {   /* another batch */
            if (tid == 0) claim[(kk + 1) & 1] = nxt;
            continue;
        }
        const bool ok = present && g53_grp_desc_ok(*ex, a.E, a.I, a.tiled);
        if (!ok) {                                           /* zero contributions */
            for (int q = tid; q < n * (MR / 4); q += 64 * NW) {
                const int j = q / (MR / 4), c = (q % (MR / 4)) * 4;
                *(float4 *)(a.contrib + (size_t)(pos0 + j) * a.E + mb * MR + c) = make_float4(0.f, 0.f, 0.f, 0.f);
            }
            if (tid == 0) claim[(kk + 1) & 1] = nxt;
            continue;
        }
        G53GrpLd<NW> ld;
#pragma unroll
        for (int j = 0; j < G53GrpLd<NW>::RPT; j++) {
            const int lp = (tid >> 3) + j * 8 * NW, piece = tid & 7;
            ld.src[j] = a.aq + (size_t)(pos0 + (lp < n ? lp : 0)) * a.I + piece * 16;
            ld.dst[j] = lp * G53_GRP_XST + piece * 16;
        }
        const size_t xps = (size_t)a.P * a.I;
        const int r0 = mb * MR + w * 32;
        const int wr = r0 + i;
        const uint8_t *arow = a.tiled ? ex->down.w + (size_t)(wr >> 3) * NKB * 1024 + (wr & 7) * 128 + g * 64
                                      : ex->down.w + (size_t)wr * a.I + g * 64;
        const int kst = a.tiled ? 1024 : 128;
        const float *s0 = (const float *)ex->down.s + (size_t)(r0 / 128) * ex->down.scols;
        g53_v16f acc[G53_GRP_NH] = {};
        if (threadIdx.x < 2 * G53_GRP_NS) flags[threadIdx.x] = 0;
        if (threadIdx.x == 0) claim[(kk + 1) & 1] = nxt;
        __syncthreads();
        int spin_err = 0;
        switch ((n + 31) >> 5) {
        case 1: g53_grp_kloop<NW, G53_GRP_NPA, NKB, 1>(acc, arow, kst, s0, s0, ld, xps, xs, flags, spin_err, lane); break;
        case 2: g53_grp_kloop<NW, G53_GRP_NPA, NKB, 2>(acc, arow, kst, s0, s0, ld, xps, xs, flags, spin_err, lane); break;
        case 3: g53_grp_kloop<NW, G53_GRP_NPA, NKB, 3>(acc, arow, kst, s0, s0, ld, xps, xs, flags, spin_err, lane); break;
        default: g53_grp_kloop<NW, G53_GRP_NPA, NKB, 4>(acc, arow, kst, s0, s0, ld, xps, xs, flags, spin_err, lane); break;
        }
        if (spin_err && lane == 0) atomicOr(&a.meta_w[1], G53_GRP_ESPIN);
#pragma unroll
        for (int h = 0; h < G53_GRP_NH; h++) {
            const int j = h * 32 + i;
            if (j >= n) continue;
            float *dst = a.contrib + (size_t)(pos0 + j) * a.E + r0 + g * 4;
#pragma unroll
            for (int q = 0; q < 4; q++)
                *(float4 *)(dst + q * 8) = make_float4(acc[h][q * 4] * a.aq_inv, acc[h][q * 4 + 1] * a.aq_inv,
                                                       acc[h][q * 4 + 2] * a.aq_inv, acc[h][q * 4 + 3] * a.aq_inv);
        }
    }
}

/* out[t][d] = (float)(sum_j (double)w[t][j] * (double)contrib[pos(t,j)][d]) (+ shared, float):
 * src/core/glm53f_ops.c:1329-1340. Four consecutive d per thread. */
__global__ void __launch_bounds__(256)
k_grp_combine(float *__restrict__ out, const float *__restrict__ contrib, const float *__restrict__ wts,
              const int *__restrict__ pos_of, int T, int E, int K, int has_sh, int *__restrict__ err,
              int *__restrict__ meta)
{
    /* the pass's error flags into the library's, and the tile count and flags cleared for the
     * next pass (every kernel that reads or sets them has finished) */
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        if (meta[1]) atomicOr(err, meta[1]);
        meta[0] = 0;
        meta[1] = 0;
    }
    const long q = (long)blockIdx.x * 256 + threadIdx.x;
    if (q * 4 >= (long)T * E) return;
    const int t = (int)(q * 4 / E), d = (int)(q * 4 % E);
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
    for (int j = 0; j < K; j++) {
        const int p = pos_of[t * (K + 1) + j];
        const double wj = (double)wts[(size_t)t * K + j];
        float4 c = make_float4(0.f, 0.f, 0.f, 0.f);
        if (p >= 0) c = *(const float4 *)(contrib + (size_t)p * E + d);
        s0 = s0 + wj * (double)c.x; s1 = s1 + wj * (double)c.y;
        s2 = s2 + wj * (double)c.z; s3 = s3 + wj * (double)c.w;
    }
    float4 o = make_float4((float)s0, (float)s1, (float)s2, (float)s3);
    if (has_sh) {
        const float4 c = *(const float4 *)(contrib + (size_t)pos_of[t * (K + 1) + K] * E + d);
        o.x = o.x + c.x; o.y = o.y + c.y; o.z = o.z + c.z; o.w = o.w + c.w;
    }
    *(float4 *)(out + (size_t)t * E + d) = o;
}

/* ------------------------------------------------------------------ dispatch ---- */
static int g_grp_mode = 1;           /* 1: T >= 2 takes this path when the shapes fit */
static uint64_t *g_grp_trace = nullptr;

/* Diagnostics: with dev_buf != NULL (device, >= gate/up items x 8 uint64), the gate/up kernel
 * records timestamps (100 MHz) of each item's phases, its CU and workgroup; NULL turns it off. */
extern "C" int g53h_set_grouped_trace(void *dev_buf)
{
    g_grp_trace = (uint64_t *)dev_buf;
    return 0;
}
static int *g_grp_err = nullptr;     /* device: accumulated error flags               */

static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

extern "C" int g53h_set_grouped(int mode)
{
    const int prev = g_grp_mode;
    g_grp_mode = mode ? 1 : 0;
    return prev;
}

/* The layer shapes this path serves (routing aside). */
static int g53_grp_shapes_ok(const G53hMoeLayer *L)
{
    if (!L) return 0;
    const float lim = L->swiglu_limit;
    const int nbe = L->hidden / 128, nbi = L->inter / 128;
    const int pow2 = (nbe & (nbe - 1)) == 0 && (nbi & (nbi - 1)) == 0;
    return L->block_c == 128 && L->hidden % 512 == 0 && L->inter % 512 == 0 && pow2 && nbe <= 32 && nbi <= 32 &&
           L->topk >= 1 && L->topk <= 16 && L->n_experts >= L->topk && L->n_experts <= 1024 && lim > 0.0f &&
           lim < 1.0e4f;
}

extern "C" int g53h_grouped_ok(const G53hMoeLayer *L)
{
    /* the grouped kernels read row-major or octet-tiled experts, not MFMA-tiled ones */
    return L && L->router && L->bias && (L->tiled == 0 || L->tiled == 1) && g53_grp_shapes_ok(L);
}

int g53h_grouped_use(const G53hMoeLayer *L, int T) { return g_grp_mode && T >= 2 && g53h_grouped_ok(L); }



extern "C" int g53h_grouped_errors(void)
{
    if (g53h_ready()) return 0;
    int v = 0;
    if (g53h_check(hipStreamSynchronize(g53h_stream()), "sync", __FILE__, __LINE__)) return -1;
    if (g53h_check(hipMemcpy(&v, g53h_errblock() + 2, 4, hipMemcpyDeviceToHost), "d2h", __FILE__, __LINE__)) return -1;
    if (v && g53h_check(hipMemset(g53h_errblock() + 2, 0, 4), "memset", __FILE__, __LINE__)) return -1;
    return v;
}

/* One planning pass of tc <= G53_GRP_MAXT tokens, in three phases: plan (sort, tiles, input
 * planes), run (the expert GEMMs for the experts present in L->experts / L->shared), combine. */
struct G53GrpPass {
    int active, tc, K, hs, maxtiles;
    int *pos_of, *meta;
    float *contrib;
    G53GrpArgs a;
};
static G53GrpPass g_pass;

static int g53_grp_plan_pass(const float *x, int tc, const G53hMoeLayer *L, const int *idx, char *ws, int *meta)
{
    const int E = L->hidden, I = L->inter, K = L->topk, NE = L->n_experts, hs = L->shared ? 1 : 0;
    const int P = tc * K + hs * tc;
    const int maxtiles = (tc * K + G53_GRP_NT - 1) / G53_GRP_NT + NE + hs * ((tc + G53_GRP_NT - 1) / G53_GRP_NT);
    hipStream_t st = g53h_stream();
    char *p = ws;
    int *tok_of = (int *)p;   p += al256((size_t)P * 4);
    int *pos_of = (int *)p;   p += al256((size_t)tc * (K + 1) * 4);
    int4 *tiles = (int4 *)p;  p += al256((size_t)maxtiles * 16);
    uint8_t *xq = (uint8_t *)p; p += al256((size_t)G53_GRP_NPX * tc * E);
    float *xinv = (float *)p; p += al256((size_t)tc * 4);
    uint8_t *aq = (uint8_t *)p; p += al256((size_t)G53_GRP_NPA * P * I);
    float *contrib = (float *)p;
    const int nch = (tc + 63) / 64;
    const size_t lds = (size_t)nch * NE * 12 + (size_t)(NE + 2) * 12;
    if (lds > 160 * 1024) return g53h_fail("g53h_moe_grouped: %zu bytes of planner LDS", lds);
    if (lds > 65536) G53_TRY(hipFuncSetAttribute((const void *)k_grp_plan, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL(k_grp_plan, dim3(1), dim3(1024), lds, st, idx, tc, K, NE, hs, tok_of, pos_of, tiles, meta,
                       I / (16 * G53_GRP_NW), E / (32 * G53_GRP_NW));
    G53_LAUNCHED("k_grp_plan");
    hipLaunchKernelGGL(k_grp_xq<G53_GRP_NPX>, dim3(tc), dim3(256), 0, st, x, E, tc, xq, xinv, L->tiled ? 1 : 0);
    G53_LAUNCHED("k_grp_xq");
    g53h_prof_mark(G53_PROF_GROUPED);
    float bound = L->swiglu_limit > 0.28f ? L->swiglu_limit : 0.28f;
    bound *= L->swiglu_limit;
    int ex = 0;
    (void)frexpf(bound, &ex);                      /* |act| <= bound < 2^ex */
    G53GrpArgs &a = g_pass.a;
    a.experts = L->experts; a.shared = L->shared; a.tiles = tiles; a.meta = meta; a.meta_w = meta; a.ctr = meta + 2;
    a.tok_of = tok_of; a.xq = xq; a.xinv = xinv; a.aq = aq; a.contrib = contrib;
    a.T = tc; a.P = P; a.E = E; a.I = I; a.NE = NE;
    a.limit = L->swiglu_limit; a.aq_scale = ldexpf(1.0f, 8 - ex); a.aq_inv = ldexpf(1.0f, ex - 8);
    a.partial = 0;
    a.tiled = L->tiled ? 1 : 0;
    a.trace = g_grp_trace;
    g_pass.active = 1; g_pass.tc = tc; g_pass.K = K; g_pass.hs = hs; g_pass.maxtiles = maxtiles;
    g_pass.pos_of = pos_of; g_pass.meta = meta; g_pass.contrib = contrib;
    return 0;
}

static int g53_grp_run_pass(const G53hExpert *experts, const G53hExpert *shared, int partial)
{
    G53GrpArgs &a = g_pass.a;
    a.experts = experts; a.shared = shared; a.partial = partial;
    const int E = a.E, I = a.I, maxtiles = g_pass.maxtiles;
    hipStream_t st = g53h_stream();
    constexpr int NW = G53_GRP_NW;
    unsigned g1 = (unsigned)((maxtiles * (I / (16 * NW)) + 7) / 8 * 8);
    unsigned g2 = (unsigned)((maxtiles * (E / (32 * NW))) + 7) / 8 * 8;
#if G53_GRP_PERS
    {
        const unsigned cap = (unsigned)(g53h_num_cus() * G53_GRP_WPC * G53_GRP_PERS) / 8 * 8;
        if (cap >= 8) { g1 = g1 < cap ? g1 : cap; g2 = g2 < cap ? g2 : cap; }
    }
#endif
#define G53_GU(N) case N: hipLaunchKernelGGL((k_grp_gateup<NW, N>), dim3(g1), dim3(64 * NW), 0, st, a); break
#define G53_DN(N) case N: hipLaunchKernelGGL((k_grp_down<NW, N>), dim3(g2), dim3(64 * NW), 0, st, a); break
    switch (E / 128) { G53_GU(4); G53_GU(8); G53_GU(16); G53_GU(32);
                       default: return g53h_fail("g53h_moe_grouped: hidden %d", E); }
    G53_LAUNCHED("k_grp_gateup");
    g53h_prof_mark(G53_PROF_GATEUP);
    switch (I / 128) { G53_DN(4); G53_DN(8); G53_DN(16); G53_DN(32);
                       default: return g53h_fail("g53h_moe_grouped: inter %d", I); }
#undef G53_GU
#undef G53_DN
    G53_LAUNCHED("k_grp_down");
    g53h_prof_mark(G53_PROF_DOWN);
    return 0;
}

static int g53_grp_combine_pass(float *out, const float *wts)
{
    hipStream_t st = g53h_stream();
    const int tc = g_pass.tc, E = g_pass.a.E;
    const long nq = (long)tc * E / 4;
    hipLaunchKernelGGL(k_grp_combine, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, st, out, g_pass.contrib, wts,
                       g_pass.pos_of, tc, E, g_pass.K, g_pass.hs, g53h_errblock() + 2, g_pass.meta);
    G53_LAUNCHED("k_grp_combine");
    g53h_prof_mark(G53_PROF_COMBINE);
    g_pass.active = 0;
    return 0;
}

static int g53_grp_chunk(float *out, const float *x, int tc, const G53hMoeLayer *L, const int *idx,
                         const float *wts, char *ws, int *meta)
{
    if (g53_grp_plan_pass(x, tc, L, idx, ws, meta) || g53_grp_run_pass(L->experts, L->shared, 0)) return -1;
    return g53_grp_combine_pass(out, wts);
}

/* Workspace of one planning pass of tc tokens. */
static size_t g53_grp_ws(const G53hMoeLayer *L, int tc)
{
    const int E = L->hidden, I = L->inter, K = L->topk, NE = L->n_experts, hs = L->shared ? 1 : 0;
    const size_t P = (size_t)tc * K + (size_t)hs * tc;
    const int maxtiles = (tc * K + G53_GRP_NT - 1) / G53_GRP_NT + NE + hs * ((tc + G53_GRP_NT - 1) / G53_GRP_NT);
    return al256(P * 4) + al256((size_t)tc * (K + 1) * 4) + al256((size_t)maxtiles * 16) +
           al256((size_t)G53_GRP_NPX * tc * E) + al256((size_t)tc * 4) + al256((size_t)G53_GRP_NPA * P * I) +
           al256(P * E * 4);
}

/* The grouped layer: router (exact), then planning passes of at most G53_GRP_MAXT tokens whose
 * 64-token masks fit the planner's LDS. idx_out / w_out receive the routing when non-NULL. */
extern "C" int g53h_moe_grouped(float *out, const float *x, int T, const G53hMoeLayer *L, int *idx_out,
                                float *w_out)
{
    if (g53h_ready()) return -1;
    if (!g53h_grouped_ok(L)) return g53h_fail("g53h_moe_grouped: layer shapes not supported");
    if (T < 0) return g53h_fail("g53h_moe_grouped: T %d", T);
    if (T == 0) return 0;
    const int K = L->topk, NE = L->n_experts;
    int tcmax = G53_GRP_MASKS / NE * 64;
    if (tcmax > G53_GRP_MAXT) tcmax = G53_GRP_MAXT;
    const int tc0 = T < tcmax ? T : tcmax;
    if (!g_grp_err) {
        G53_TRY(hipMalloc((void **)&g_grp_err, 256));
        G53_TRY(hipMemset(g_grp_err, 0, 256));
    }
    const size_t rsz = al256((size_t)2 * T * NE * 4), isz = al256((size_t)T * K * 4);
    char *ws = (char *)g53h_workspace(rsz + 2 * isz + g53_grp_ws(L, tc0));
    if (!ws) return -1;
    int *idx = idx_out ? idx_out : (int *)(ws + rsz);
    float *w = w_out ? w_out : (float *)(ws + rsz + isz);
    g53h_prof_mark(G53_PROF_START);
    if (g53h_router_into(idx, w, x, T, L->router, L->router_dt, L->bias, NE, L->hidden, K, L->norm_topk,
                         L->routed_scale, nullptr, (float *)ws, nullptr, nullptr, nullptr))
        return -1;
    g53h_prof_mark(G53_PROF_ROUTER);
    int *meta = g_grp_err + 16;                    /* [0] tiles, [1] flags; zero between calls */
    for (int t0 = 0; t0 < T; t0 += tc0) {
        const int tc = T - t0 < tc0 ? T - t0 : tc0;
        if (g53_grp_chunk(out + (size_t)t0 * L->hidden, x + (size_t)t0 * L->hidden, tc, L, idx + (size_t)t0 * K,
                          w + (size_t)t0 * K, ws + rsz + 2 * isz, meta))
            return -1;
    }
    return 0;
}

/* ------------------------------------------------------------- phased entry ---- */
static int g53_grp_tcmax(int NE)
{
    int tcmax = G53_GRP_MASKS / NE * 64;
    return tcmax > G53_GRP_MAXT ? G53_GRP_MAXT : tcmax;
}

extern "C" int g53h_grouped_max_tokens(const G53hMoeLayer *L)
{
    if (!g_grp_mode || !g53_grp_shapes_ok(L)) return 0;
    return g53_grp_tcmax(L->n_experts);
}

extern "C" int g53h_grouped_begin(const float *x, int T, const G53hMoeLayer *L, const int *idx)
{
    if (g53h_ready()) return -1;
    if (!g53_grp_shapes_ok(L)) return g53h_fail("g53h_grouped_begin: layer shapes not supported");
    if (T < 1 || T > g53_grp_tcmax(L->n_experts)) return g53h_fail("g53h_grouped_begin: T %d", T);
    if (!g_grp_err) {
        G53_TRY(hipMalloc((void **)&g_grp_err, 256));
        G53_TRY(hipMemset(g_grp_err, 0, 256));
    }
    char *ws = (char *)g53h_workspace(g53_grp_ws(L, T));
    if (!ws) return -1;
    return g53_grp_plan_pass(x, T, L, idx, ws, g_grp_err + 16);
}

extern "C" int g53h_grouped_batch(const G53hMoeLayer *L)
{
    if (!g_pass.active) return g53h_fail("g53h_grouped_batch: no pass begun");
    if (L && (L->tiled ? 1 : 0) != g_pass.a.tiled)
        return g53h_fail("g53h_grouped_batch: the pass was planned for %s experts", g_pass.a.tiled ? "octet-tiled" : "row-major");
    if (!L || L->n_experts != g_pass.a.NE || L->hidden != g_pass.a.E || L->inter != g_pass.a.I)
        return g53h_fail("g53h_grouped_batch: another layer than the pass's");
    if (L->shared && !g_pass.hs) return g53h_fail("g53h_grouped_batch: the pass was planned without a shared expert");
    return g53_grp_run_pass(L->experts, L->shared, 1);
}

extern "C" int g53h_grouped_end(float *out, const float *wts)
{
    if (!g_pass.active) return g53h_fail("g53h_grouped_end: no pass begun");
    return g53_grp_combine_pass(out, wts);
}
