/* g53h_ops.hip - the expert path's building blocks on gfx950, bit-exact with the reference:
 *
 *   k_mm_f8_generic   FP8 block-scaled (or int4) matvec for any shape (ragged blocks, any
 *                     br/bc), one thread per (token, row): the unit-level glm53f_mm. The
 *                     layer paths use the kernels of g53h_moe.hip, g53h_rows.hip and the
 *                     decode files.
 *   k_swiglu          clamped SwiGLU.
 *   k_router_scores   sigmoid(W x) and sigmoid + bias for T tokens, one wave per expert.
 *   k_router_select_w top-k by repeated argmax (strict >, lowest index), renormalise, scale.
 *   k_route_topn      next-layer prediction.
 */
#include <hip/hip_runtime.h>
#include <math.h>

#include "g53h.h"
#include "g53h_core.h"
#include "g53h_kern.h"
#include "g53h_runtime.h"

/* ------------------------------------------------------------- FP8 matvec ---- */
#include "g53h_rowdot.h"

__device__ float g53_row_dot_i4(const G53hMat &m, int o, const float *x)
{
    const uint8_t *row = m.w + (size_t)o * (m.cols / 2);
    const float *srow = m.s + (size_t)o * m.scols;
    double acc = 0.0;
    for (int g = 0, j0 = 0; j0 < m.cols; g++, j0 += m.bc) {
        const int j1 = (j0 + m.bc < m.cols) ? j0 + m.bc : m.cols;
        const double p = g53_group_dot_i4(row, x, j0, j1) * (double)srow[g];
        acc = acc + p;
    }
    return (float)acc;
}

__device__ float g53_row_dot(const G53hMat &m, int o, const float *x)
{
    if (m.flags & G53H_MAT_I4) return g53_row_dot_i4(m, o, x);
    const uint8_t *row = m.w + (size_t)o * m.cols;
    const float *srow = m.s + (size_t)(o / m.br) * m.scols;
    double acc = 0.0;
    for (int b = 0, j0 = 0; j0 < m.cols; b++, j0 += m.bc) {
        const int j1 = (j0 + m.bc < m.cols) ? j0 + m.bc : m.cols;
        const double bsum = g53_block_dot(row, x, j0, j1);
        const double p = bsum * (double)srow[b];
        acc = acc + p;
    }
    return (float)acc;
}

__global__ void k_mm_f8_generic(float *__restrict__ y, const float *__restrict__ x, int T, G53hMat m)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)T * m.rows) return;
    const int t = (int)(i / m.rows), o = (int)(i % m.rows);
    y[(size_t)t * m.rows + o] = g53_row_dot(m, o, x + (size_t)t * m.cols);
}

extern "C" int g53h_mm_f8(float *y, const float *x, int T, const G53hMat *m)
{
    if (g53h_ready()) return -1;
    if (T <= 0) return 0;
    if (!m || !m->w || !m->s) return g53h_fail("g53h_mm_f8: unbound matrix");
    if (m->rows <= 0 || m->cols <= 0 || m->br <= 0 || m->bc <= 0 ||
        m->scols != (m->cols + m->bc - 1) / m->bc || ((m->flags & G53H_MAT_I4) && (m->cols & 1)))
        return g53h_fail("g53h_mm_f8: bad geometry %dx%d block %dx%d scols %d", m->rows, m->cols,
                         m->br, m->bc, m->scols);
    if (m->flags & G53H_MAT_TILED) return g53h_fail("g53h_mm_f8: octet-tiled codes are read by the decode kernel only");
    const long n = (long)T * m->rows;
    hipLaunchKernelGGL(k_mm_f8_generic, dim3((unsigned)((n + 127) / 128)), dim3(128), 0,
                       g53h_stream(), y, x, T, *m);
    G53_LAUNCHED("k_mm_f8_generic");
    return 0;
}

/* ----------------------------------------------------------------- SwiGLU ---- */
__global__ void k_swiglu(float *__restrict__ y, const float *__restrict__ gu, int n, int T, float limit)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)n * T) return;
    const int t = (int)(i / n), k = (int)(i % n);
    const float *g = gu + (size_t)t * 2 * n;
    y[i] = g53_swiglu1(g[k], g[n + k], limit);
}

extern "C" int g53h_swiglu(float *y, const float *gu, int n, int T, float limit)
{
    if (g53h_ready()) return -1;
    const long m = (long)n * T;
    if (m <= 0) return 0;
    hipLaunchKernelGGL(k_swiglu, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, g53h_stream(), y,
                       gu, n, T, limit);
    G53_LAUNCHED("k_swiglu");
    return 0;
}

/* Swiglu over separate gate/up slot outputs: g, u [rows_total][n] -> y. */
__global__ void k_swiglu_split(float *__restrict__ y, const float *__restrict__ g,
                               const float *__restrict__ u, long m, float limit)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < m) y[i] = g53_swiglu1(g[i], u[i], limit);
}

int g53h_swiglu_split(float *y, const float *g, const float *u, long m, float limit)
{
    if (m <= 0) return 0;
    hipLaunchKernelGGL(k_swiglu_split, dim3((unsigned)((m + 255) / 256)), dim3(256), 0,
                       g53h_stream(), y, g, u, m, limit);
    G53_LAUNCHED("k_swiglu_split");
    return 0;
}

#include "g53h_gemv.h"

/* scores[t][e] = sigmoid(dot); choice[t][e] = score + bias[e]. One wave per (token, expert),
 * one wave per workgroup so the experts spread over every CU. */
__global__ void __launch_bounds__(64) k_router_scores(float *__restrict__ score, float *__restrict__ choice,
                                                      const float *__restrict__ x, int T,
                                                      const void *__restrict__ gate, int dt,
                                                      const float *__restrict__ bias, int NE, int E)
{
    const int lane = threadIdx.x;
    const int e = blockIdx.x, t = blockIdx.y;
    const float d = g53_router_dot(gate, dt, e, E, x + (size_t)t * E, lane);
    if (lane == 0) {
        const float s = g53_sigmoidf(d);
        score[(size_t)t * NE + e] = s;
        if (choice) choice[(size_t)t * NE + e] = s + bias[e];
    }
}

/* The same scores for many tokens on the FP64 matrix cores (v_mfma_f64_16x16x4f64). Every
 * product (double)bf16 * (double)x is exact in double, as in k_router_scores; the instruction
 * adds them with double FMAs, in an order of its own. A workgroup computes the 16 x 16 tile of
 * experts e0 = 16 * blockIdx.x .. +15 and tokens t0 = 16 * blockIdx.y .. +15; its four waves
 * split the columns (wave w takes columns 64w .. 64w+63 of every 256-column chunk) and their
 * partial sums are added in LDS at the end. Operands: lane l gives A[l % 16][l / 16] (an
 * expert's weight) and B[l / 16][l % 16] (a token's x); step s uses column 64w + 16(l/16) + s
 * of the chunk, so a lane reads 32 consecutive router bytes per chunk. Result: lane l, register
 * r holds C[4r + l/16][l % 16]. x chunks are staged in LDS. bf16 router rows, E a multiple of
 * 256. */
typedef double g53_v4d __attribute__((ext_vector_type(4)));
#ifndef G53_RM32_S
#define G53_RM32_S    8         /* column ranges of the large-batch router               */
#endif
static_assert(G53_RM32_S >= 1 && G53_RM32_S <= 8, "the selection sums at most 8 column ranges");
#ifndef G53_RM32_MINT
#define G53_RM32_MINT 512       /* tokens from which the large-batch router is used       */
#endif
#define G53_RM_XST 260                                  /* LDS floats per token row       */
__global__ void __launch_bounds__(256) k_router_mfma(float *__restrict__ score, float *__restrict__ choice,
                                                     const float *__restrict__ x, int T,
                                                     const uint16_t *__restrict__ gate,
                                                     const float *__restrict__ bias, int NE, int E, int klen,
                                                     double *__restrict__ psum)
{
    __shared__ __attribute__((aligned(16))) float xs[16 * G53_RM_XST];
    __shared__ g53_v4d part[3][64];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t0 = blockIdx.y * 16, e0 = blockIdx.x * 16;
    const int i = lane & 15, g = lane >> 4;
    const int er = e0 + i < NE ? e0 + i : NE - 1;          /* rows past NE: discarded       */
    const uint16_t *wrow = gate + (size_t)er * E + w * 64 + g * 16;
    const float *xl = xs + i * G53_RM_XST + w * 64 + g * 16;
    g53_v4d acc = {0.0, 0.0, 0.0, 0.0};
    const int kb = blockIdx.z * klen;                        /* this workgroup's column range */
    for (int k0 = kb; k0 < kb + klen; k0 += 256) {
        const uint4 wv0 = *(const uint4 *)(wrow + k0), wv1 = *(const uint4 *)(wrow + k0 + 8);
        __syncthreads();
        for (int q = threadIdx.x; q < 16 * 64; q += 256) {
            const int tk = q >> 6, c = (q & 63) * 4;
            const int tt = t0 + tk < T ? t0 + tk : T - 1;
            *(float4 *)(xs + tk * G53_RM_XST + c) = *(const float4 *)(x + (size_t)tt * E + k0 + c);
        }
        __syncthreads();
        const uint32_t d[8] = {wv0.x, wv0.y, wv0.z, wv0.w, wv1.x, wv1.y, wv1.z, wv1.w};
#pragma unroll
        for (int k = 0; k < 8; k++) {
            acc = __builtin_amdgcn_mfma_f64_16x16x4f64((double)g53_bitsf(d[k] << 16), (double)xl[2 * k], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f64_16x16x4f64((double)g53_bitsf(d[k] & 0xffff0000u), (double)xl[2 * k + 1],
                                                       acc, 0, 0, 0);
        }
    }
    if (w > 0) part[w - 1][lane] = acc;
    __syncthreads();
    if (w > 0) return;
    acc = acc + part[0][lane] + part[1][lane] + part[2][lane];
    const int t = t0 + i;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int e = e0 + 4 * r + g;
        if (t < T && e < NE && psum) {                        /* a column range: its sum */
            psum[((size_t)blockIdx.z * T + t) * NE + e] = acc[r];
        } else if (t < T && e < NE) {
            const float s = g53_sigmoidf((float)acc[r]);
            score[(size_t)t * NE + e] = s;
            if (choice) choice[(size_t)t * NE + e] = s + bias[e];
        }
    }
}

/* The same partial sums for large batches: one wave per workgroup owns a 32 x 32 tile
 * (experts e0 = 32 * bx .., tokens t0 = 32 * by ..) over the column range bz * klen .. + klen, as 2 x 2 blocks of v_mfma_f64_16x16x4f64, so that each operand
 * converted to double feeds two instructions. Both operands come straight from memory (L2):
 * per 64-column chunk, lane l reads 16 consecutive columns 16 (l / 16) .. of its two expert rows
 * (l % 16, 16 + l % 16) and of its two token rows; step s of the chunk uses column
 * 16 (l / 16) + s, the same K assignment for A and B. The next chunk's loads are issued before
 * the current chunk's arithmetic. The sums go to psum[bz][t][e]; the selection kernel adds
 * the ranges in column order. bf16 router rows, klen a multiple of 64. */
__global__ void __launch_bounds__(64) k_router_mfma32(const float *__restrict__ x, int T,
                                                      const uint16_t *__restrict__ gate, int NE, int E,
                                                      int klen, int S, double *__restrict__ psum)
{
    /* workgroups are dealt round-robin over the 8 XCDs: XCD x takes the contiguous tile range
     * x * per .., expert tiles fastest, so the expert tiles that read one token tile's
     * activations share one L2 */
    const int ET = (NE + 31) >> 5, TT = (T + 31) >> 5, n = ET * TT * S, per = (int)(gridDim.x >> 3);
    const int j = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
    if (j >= n) return;
    const int bx = j % ET, by = (j / ET) % TT, bz = j / (ET * TT);
    const int lane = threadIdx.x, i = lane & 15, g = lane >> 4;
    const int e0 = bx * 32, t0 = by * 32;
    const int kb = bz * klen;
    const uint16_t *wr[2];
    const float *xr[2];
#pragma unroll
    for (int f = 0; f < 2; f++) {
        const int e = min(e0 + 16 * f + i, NE - 1), t = min(t0 + 16 * f + i, T - 1);   /* past the end: discarded */
        wr[f] = gate + (size_t)e * E + kb + 16 * g;
        xr[f] = x + (size_t)t * E + kb + 16 * g;
    }
    g53_v4d acc[2][2] = {};
    uint4 wa[2][2], wb[2][2];
    float4 xa[2][4], xb[2][4];
#define G53_RM32_LD(W, X, c) do { _Pragma("unroll") for (int f = 0; f < 2; f++) {                               \
        W[f][0] = *(const uint4 *)(wr[f] + (c)); W[f][1] = *(const uint4 *)(wr[f] + (c) + 8);                   \
        _Pragma("unroll") for (int q = 0; q < 4; q++) X[f][q] = *(const float4 *)(xr[f] + (c) + 4 * q); } } while (0)
#define G53_RM32_MUL(W, X) do {                                                                                 \
        _Pragma("unroll") for (int s = 0; s < 16; s++) {                                                        \
            double a[2], b[2];                                                                                  \
            _Pragma("unroll") for (int f = 0; f < 2; f++) {                                                     \
                const uint32_t wd = ((const uint32_t *)&W[f][s >> 3])[(s & 7) >> 1];                            \
                a[f] = (double)g53_bitsf((s & 1) ? (wd & 0xffff0000u) : (wd << 16));                            \
                b[f] = (double)((const float *)&X[f][s >> 2])[s & 3];                                           \
            }                                                                                                   \
            _Pragma("unroll") for (int f = 0; f < 2; f++)                                                       \
                _Pragma("unroll") for (int h = 0; h < 2; h++)                                                   \
                    acc[f][h] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[f], b[h], acc[f][h], 0, 0, 0);           \
        } } while (0)
    G53_RM32_LD(wa, xa, 0);
    for (int c = 0; c < klen; c += 128) {
        if (c + 64 < klen) G53_RM32_LD(wb, xb, c + 64);
        G53_RM32_MUL(wa, xa);
        if (c + 64 >= klen) break;
        if (c + 128 < klen) G53_RM32_LD(wa, xa, c + 128);
        G53_RM32_MUL(wb, xb);
    }
#undef G53_RM32_LD
#undef G53_RM32_MUL
#pragma unroll
    for (int f = 0; f < 2; f++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int t = t0 + 16 * h + i;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int e = e0 + 16 * f + 4 * r + g;
                if (t < T && e < NE) psum[((size_t)bz * T + t) * NE + e] = acc[f][h][r];
            }
        }
}

extern "C" __device__ unsigned __ockl_wfred_max_u32(unsigned);

/* Top-k and weights of each token: one wave per token, four per workgroup, and the top-k as K
 * rounds of arg-max over keys each lane holds sorted (the reference's rounds of "first
 * strictly greater", src/core/glm53f_ops.c:957-969: the larger choice first, the lower index
 * among equal ones, NaN and -inf never). With part != NULL the logits are first summed from
 * the S column ranges in column order and the scores and choices written. A token with fewer
 * than K selectable experts gets index 0 with expert 0's score in the missing slots and sets
 * *nan_flag (the reference aborts there). Then the weights: the unbiased scores of the chosen
 * experts, renormalised in double if norm_topk (:970-975), times routed_scale. When experts !=
 * NULL the chosen experts' descriptors (and the shared expert's) are copied to slots[t][*], so
 * the expert kernels find their matrices with one load. NE <= 64 * NV. */
template <int NV>
__device__ __forceinline__ void g53_select_token(int t, int lane, int *__restrict__ idx, float *__restrict__ w,
                                                 float *__restrict__ score, float *__restrict__ choice,
                                                 const double *__restrict__ part, int S,
                                                 const float *__restrict__ bias, int T, int NE, int K,
                                                 int norm_topk, float routed_scale, int *__restrict__ nan_flag,
                                                 int set_flag, const G53hExpert *__restrict__ experts,
                                                 const G53hExpert *__restrict__ shared,
                                                 G53hExpert *__restrict__ slots)
{
    uint32_t key[NV];
    int vid[NV];
    float vsc[NV];
    double d[NV];
    if (part) {
        const int ec = NE - 1;
        if constexpr (NV <= 8) {                              /* every range's loads in flight at once */
            double pv[8][NV];
#pragma unroll
            for (int q = 0; q < 8; q++)
#pragma unroll
                for (int v = 0; v < NV; v++)
                    pv[q][v] = part[((size_t)min(q, S - 1) * T + t) * NE + min(lane + 64 * v, ec)];
#pragma unroll
            for (int v = 0; v < NV; v++) {
                d[v] = pv[0][v];
#pragma unroll
                for (int q = 1; q < 8; q++)
                    if (q < S) d[v] = d[v] + pv[q][v];
            }
        } else {                                              /* range by range: NV loads in flight */
#pragma unroll
            for (int v = 0; v < NV; v++) d[v] = part[(size_t)t * NE + min(lane + 64 * v, ec)];
            for (int q = 1; q < S; q++)
#pragma unroll
                for (int v = 0; v < NV; v++) d[v] = d[v] + part[((size_t)q * T + t) * NE + min(lane + 64 * v, ec)];
        }
    }
#pragma unroll
    for (int v = 0; v < NV; v++) {
        const int e = lane + 64 * v;
        float sc = 0.0f, ch = -INFINITY;
        if (e < NE) {
            const size_t o = (size_t)t * NE + e;
            if (part) {
                sc = g53_sigmoidf((float)d[v]);
                ch = sc + bias[e];
                score[o] = sc;
                choice[o] = ch;
            } else {
                sc = score[o];
                ch = choice[o];
            }
        }
        key[v] = (ch > -INFINITY) ? g53_fkey(ch) : 0u;        /* 0: never chosen */
        vid[v] = e;
        vsc[v] = sc;
    }
    const float sc0 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(vsc[0]), 0));   /* expert 0's */
    /* each lane sorts its keys, largest first, the lower index first among equal keys */
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
    int pos = 0, my_e = 0;                                    /* lane j keeps round j's winner */
    float my_s = sc0;
    for (int j = 0; j < K; j++) {
        const uint32_t m = __ockl_wfred_max_u32(key[0]);
        if (m == 0) break;                                    /* fewer than K selectable */
        const uint64_t cand = __ballot(key[0] == m);
        int win;
        if (__popcll(cand) == 1) win = (int)__builtin_ctzll(cand);
        else win = (int)(__ockl_wfred_min_u32(key[0] == m ? (uint32_t)vid[0] : 0xffffffffu) & 63);
        const int e = __builtin_amdgcn_readlane(vid[0], win);
        const float ws = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(vsc[0]), win));
        if (lane == j) { my_e = e; my_s = ws; }
        const bool me = lane == win;                          /* the winner shifts its list */
#pragma unroll
        for (int q = 0; q + 1 < NV; q++) {
            key[q] = me ? key[q + 1] : key[q];
            vid[q] = me ? vid[q + 1] : vid[q];
            vsc[q] = me ? vsc[q + 1] : vsc[q];
        }
        key[NV - 1] = me ? 0u : key[NV - 1];
        pos++;
    }
    if (lane == 0 && nan_flag) {
        if (set_flag) *nan_flag = pos < K;                    /* one token: the flag's only writer */
        else if (pos < K) atomicOr(nan_flag, 1);
    }
    float wj = my_s;
    if (norm_topk) {
        double sum = 0.0;
        for (int j = 0; j < K; j++) sum += (double)__uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(my_s), j));
        wj = (float)((double)my_s / (sum + 1e-20));
    }
    if (lane < K) {
        idx[(size_t)t * K + lane] = my_e;
        w[(size_t)t * K + lane] = wj * routed_scale;
    }
    if (experts) {
        const int nslots = K + (shared ? 1 : 0);
        const int words = (int)(sizeof(G53hExpert) / 4);
        for (int q = lane; q < nslots * words; q += 64) {
            const int j = q / words, k = q % words;
            const int ej = __shfl(my_e, j < K ? j : 0);
            const G53hExpert *src = j < K ? &experts[ej] : shared;
            ((int *)&slots[(size_t)t * nslots + j])[k] = ((const int *)src)[k];
        }
    }
}

template <int NV>
__global__ void __launch_bounds__(256) k_router_select_w(int *__restrict__ idx, float *__restrict__ w,
                                                         float *__restrict__ score, float *__restrict__ choice,
                                                         const double *__restrict__ part, int S,
                                                         const float *__restrict__ bias, int T, int NE, int K,
                                                         int norm_topk, float routed_scale,
                                                         int *__restrict__ nan_flag,
                                                         const G53hExpert *__restrict__ experts,
                                                         const G53hExpert *__restrict__ shared,
                                                         G53hExpert *__restrict__ slots)
{
    const int lane = threadIdx.x & 63;
    const int t = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (t >= T) return;
    g53_select_token<NV>(t, lane, idx, w, score, choice, part, S, bias, T, NE, K, norm_topk, routed_scale, nan_flag,
                         0, experts, shared, slots);
}

/* slots[t][j] = experts[idx[t][j]] (j < K), slots[t][K] = *shared: the descriptor table of
 * the expert kernels, for callers that route elsewhere. */
__global__ void k_resolve_slots(G53hExpert *__restrict__ slots, const G53hExpert *__restrict__ experts,
                                const int *__restrict__ idx, const G53hExpert *__restrict__ shared, int T,
                                int K, int nslots)
{
    const int words = (int)(sizeof(G53hExpert) / 4);
    const long q = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= (long)T * nslots * words) return;
    const int k = (int)(q % words), j = (int)((q / words) % nslots), t = (int)(q / ((long)words * nslots));
    const G53hExpert *src = j < K ? &experts[idx[(size_t)t * K + j]] : shared;
    ((int *)&slots[(size_t)t * nslots + j])[k] = ((const int *)src)[k];
}

int g53h_resolve_slots(G53hExpert *slots, const G53hExpert *experts, const int *idx, const G53hExpert *shared,
                       int T, int K)
{
    const int nslots = K + (shared ? 1 : 0);
    const long n = (long)T * nslots * (long)(sizeof(G53hExpert) / 4);
    hipLaunchKernelGGL(k_resolve_slots, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, g53h_stream(), slots,
                       experts, idx, shared, T, K, nslots);
    G53_LAUNCHED("k_resolve_slots");
    return 0;
}

/* Library-owned buffer of the split router's partial sums (grown as needed, kept). */
static void *g_router_part = nullptr;
static size_t g_router_part_bytes = 0;
static void *g53_router_part(size_t bytes)
{
    if (bytes <= g_router_part_bytes) return g_router_part;
    if (g_router_part) {
        if (hipStreamSynchronize(g53h_stream()) != hipSuccess || hipFree(g_router_part) != hipSuccess) {
            g53h_fail("g53h_router: cannot release the partial-sum buffer");
            return nullptr;
        }
        g_router_part = nullptr;
        g_router_part_bytes = 0;
    }
    if (hipMalloc(&g_router_part, bytes) != hipSuccess) {
        (void)hipGetLastError();
        g53h_fail("g53h_router: cannot allocate %zu bytes of partial sums", bytes);
        return nullptr;
    }
    g_router_part_bytes = bytes;
    return g_router_part;
}

int g53h_router_into(int *idx, float *w, const float *x, int T, const void *gate, int gate_dt,
                     const float *bias, int NE, int E, int K, int norm_topk, float routed_scale,
                     int *nan_flag, float *scratch, const G53hExpert *experts, const G53hExpert *shared,
                     G53hExpert *slots)
{
    if (NE < 1 || NE > 1024) return g53h_fail("g53h_router: %d experts (max 1024)", NE);
    if (K < 1 || K > NE || K > GLM53F_MAX_TOPK_DEV) return g53h_fail("g53h_router: topk %d", K);
    float *score = scratch, *choice = scratch + (size_t)T * NE;
    const double *psum = nullptr;                            /* split logits, summed by the selection */
    int nsum = 1;
    if (T >= G53_RM32_MINT && gate_dt == 1 && E % (64 * G53_RM32_S) == 0) {   /* large batches */
        const int S = G53_RM32_S;
        double *part = (double *)g53_router_part((size_t)S * T * NE * sizeof(double));
        if (!part) return -1;
        const unsigned n32 = (unsigned)(((NE + 31) / 32) * ((T + 31) / 32) * S + 7) / 8 * 8;
        hipLaunchKernelGGL(k_router_mfma32, dim3(n32), dim3(64), 0, g53h_stream(), x, T, (const uint16_t *)gate, NE,
                           E, E / S, S, part);
        G53_LAUNCHED("k_router_mfma32");
        psum = part;
        nsum = S;
    } else if (T >= 2 && gate_dt == 1 && E % 256 == 0) {    /* batches: the matrix-core form */
        /* few tiles (small T): the columns are split over up to 8 workgroups per tile so that
         * enough loads are in flight; the partial sums are added in column order after */
        const int tiles = ((NE + 15) / 16) * ((T + 15) / 16);
        int S = 1;
        while (S < 8 && tiles * S * 2 <= 640 && (E / (S * 2)) % 256 == 0) S *= 2;
        double *part = nullptr;
        if (S > 1) {
            part = (double *)g53_router_part((size_t)S * T * NE * sizeof(double));
            if (!part) return -1;
        }
        hipLaunchKernelGGL(k_router_mfma, dim3((NE + 15) / 16, (T + 15) / 16, S), dim3(256), 0, g53h_stream(),
                           score, choice, x, T, (const uint16_t *)gate, bias, NE, E, E / S, part);
        G53_LAUNCHED("k_router_mfma");
        if (S > 1) { psum = part; nsum = S; }
    } else {
        hipLaunchKernelGGL(k_router_scores, dim3(NE, T), dim3(64), 0, g53h_stream(), score, choice, x, T, gate,
                           gate_dt, bias, NE, E);
        G53_LAUNCHED("k_router_scores");
    }
    /* the selection, after the sum of the column ranges when the logits were split */
    const dim3 gs((unsigned)((T + 3) / 4));
    if (NE <= 320)
        hipLaunchKernelGGL(k_router_select_w<5>, gs, dim3(256), 0, g53h_stream(), idx, w, score, choice, psum, nsum,
                           bias, T, NE, K, norm_topk, routed_scale, nan_flag, experts, shared, slots);
    else
        hipLaunchKernelGGL(k_router_select_w<16>, gs, dim3(256), 0, g53h_stream(), idx, w, score, choice, psum, nsum,
                           bias, T, NE, K, norm_topk, routed_scale, nan_flag, experts, shared, slots);
    G53_LAUNCHED("k_router_select_w");
    return 0;
}

extern "C" int g53h_router(int *idx, float *w, const float *x, int T, const void *gate, int gate_dt,
                           const float *bias, int NE, int E, int K, int norm_topk,
                           float routed_scale, int *nan_flag)
{
    if (g53h_ready()) return -1;
    if (T <= 0) return 0;
    float *ws = (float *)g53h_workspace((size_t)2 * T * (NE > 0 ? NE : 1) * sizeof(float));
    if (!ws) return -1;
    return g53h_router_into(idx, w, x, T, gate, gate_dt, bias, NE, E, K, norm_topk, routed_scale,
                            nan_flag, ws, nullptr, nullptr, nullptr);
}


/* Wave-wide argmax with the reference's rule: strictly greater wins, so the lowest index among
 * equal maxima; an empty candidate (index < 0) never wins. */
__device__ inline void g53_argmax_merge(float &bv, int &bi, float ov, int oi)
{
    if (oi < 0) return;
    if (bi < 0 || ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}

__global__ void __launch_bounds__(64) k_route_topn(int *__restrict__ idx, int n,
                                                   const float *__restrict__ choice, int NE,
                                                   const float *__restrict__ score, float *__restrict__ score_out)
{
    g53_topn_token((int)blockIdx.x, (int)threadIdx.x, idx, n, choice, NE, score, score_out);
}

/* One decode token's routing and next-layer prediction in two launches: the scores of both
 * routers (blockIdx.y 0: this layer's, 1: the next layer's), then workgroup 0 selects the top-k
 * with weights and writes the NaN flag (0 or 1), workgroup 1 the next layer's top-n. */
__global__ void __launch_bounds__(64) k_router_scores2(float *__restrict__ sc0, float *__restrict__ ch0,
                                                       const void *__restrict__ g0, int dt0,
                                                       const float *__restrict__ b0,
                                                       float *__restrict__ sc1, float *__restrict__ ch1,
                                                       const void *__restrict__ g1, int dt1,
                                                       const float *__restrict__ b1, const float *__restrict__ x,
                                                       int NE, int E)
{
    const int lane = threadIdx.x, e = blockIdx.x, which = blockIdx.y;
    const float d = g53_router_dot(which ? g1 : g0, which ? dt1 : dt0, e, E, x, lane);
    if (lane == 0) {
        const float s = g53_sigmoidf(d);
        (which ? sc1 : sc0)[e] = s;
        (which ? ch1 : ch0)[e] = s + (which ? b1 : b0)[e];
    }
}

template <int NV>
__global__ void __launch_bounds__(128) k_route_decode(int *__restrict__ idx, float *__restrict__ w,
                                                      int *__restrict__ nan_flag, float *__restrict__ score,
                                                      float *__restrict__ choice, const float *__restrict__ bias,
                                                      int NE, int K, int norm_topk, float routed_scale,
                                                      int *__restrict__ pred, int n, const float *__restrict__ nscore,
                                                      const float *__restrict__ nchoice, unsigned *__restrict__ mb,
                                                      int mb_slot, int mb_off_w, unsigned seq)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (wave == 0)
        g53_select_token<NV>(0, lane, idx, w, score, choice, nullptr, 1, bias, 1, NE, K, norm_topk, routed_scale,
                             nan_flag, 1, nullptr, nullptr, nullptr);
    else if (n > 0)
        g53_topn_token(0, lane, pred, n, nchoice, NE, nscore, nullptr);
    if (!mb) return;
    /* the host's copy: idx [K], the flag, pred [n], then the sequence word */
    __threadfence_block();
    __syncthreads();
    unsigned *d = mb + mb_off_w;
    for (int i = threadIdx.x; i < K + 1 + n; i += 128)
        d[i] = (unsigned)(i < K ? idx[i] : i == K ? nan_flag[0] : pred[i - K - 1]);
    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(mb + mb_slot, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

/* The prefill prediction's vote (src/core/glm53f_ops.c:1206-1225): the experts named in ids
 * [T][n] ordered by how many tokens named them, most first, ties in the order of their first
 * appearance (t, then j). out[0] = the number of distinct experts, out[1 + r] = the expert of
 * rank r. One workgroup: counts and first positions in LDS, then each expert's rank counted
 * against every other. */
__global__ void __launch_bounds__(1024) k_vote(int *__restrict__ out, const int *__restrict__ ids, int T, int n,
                                               int NE)
{
    __shared__ int votes[1024], first[1024];
    for (int e = threadIdx.x; e < NE; e += 1024) { votes[e] = 0; first[e] = 0x7fffffff; }
    __syncthreads();
    for (int q = threadIdx.x; q < T * n; q += 1024) {
        const int e = ids[q];
        if (e < 0 || e >= NE) continue;
        atomicAdd(&votes[e], 1);
        atomicMin(&first[e], q);
    }
    __syncthreads();
    int distinct = 0;
    for (int e = threadIdx.x; e < NE; e += 1024) {                   /* NE <= 1024 */
        const int v = votes[e];
        if (!v) continue;
        const int f = first[e];
        int r = 0;
        for (int o = 0; o < NE; o++) {
            const int vo = votes[o];
            r += vo > v || (vo == v && vo && first[o] < f);
        }
        out[1 + r] = e;
    }
    if (threadIdx.x < NE) distinct = votes[threadIdx.x] != 0;        /* NE <= 1024: one each */
    const int total = __syncthreads_count(distinct);
    if (threadIdx.x == 0) out[0] = total;
}

extern "C" int g53h_route_topn(int *idx, int n, const float *x, const void *gate, int gate_dt,
                               const float *bias, int NE, int E)
{
    if (g53h_ready()) return -1;
    if (n <= 0) return 0;
    if (NE < 1 || NE > 64 * G53_SEL_PER_LANE) return g53h_fail("g53h_route_topn: %d experts", NE);
    float *ws = (float *)g53h_workspace((size_t)2 * NE * sizeof(float));
    if (!ws) return -1;
    hipLaunchKernelGGL(k_router_scores, dim3(NE, 1), dim3(64), 0, g53h_stream(), ws + NE, ws, x, 1, gate,
                       gate_dt, bias, NE, E);
    G53_LAUNCHED("k_router_scores");
    hipLaunchKernelGGL(k_route_topn, dim3(1), dim3(64), 0, g53h_stream(), idx, n, ws, NE, ws + NE, nullptr);
    G53_LAUNCHED("k_route_topn");
    return 0;
}

extern "C" int g53h_route_topn_batch(int *idx, float *score_out, int n, const float *x, int T, const void *gate,
                                     int gate_dt, const float *bias, int NE, int E)
{
    if (g53h_ready()) return -1;
    if (n <= 0 || T <= 0) return 0;
    if (NE < 1 || NE > 64 * G53_SEL_PER_LANE) return g53h_fail("g53h_route_topn_batch: %d experts", NE);
    if (n > NE) return g53h_fail("g53h_route_topn_batch: %d of %d experts", n, NE);
    float *ws = (float *)g53h_workspace((size_t)2 * T * NE * sizeof(float));
    if (!ws) return -1;
    float *choice = ws, *score = ws + (size_t)T * NE;
    hipLaunchKernelGGL(k_router_scores, dim3(NE, T), dim3(64), 0, g53h_stream(), score, choice, x, T, gate,
                       gate_dt, bias, NE, E);
    G53_LAUNCHED("k_router_scores");
    hipLaunchKernelGGL(k_route_topn, dim3(T), dim3(64), 0, g53h_stream(), idx, n, choice, NE, score, score_out);
    G53_LAUNCHED("k_route_topn");
    return 0;
}

extern "C" int g53h_vote(int *out, const int *ids, int T, int n, int NE)
{
    if (g53h_ready()) return -1;
    if (NE < 1 || NE > 1024) return g53h_fail("g53h_vote: %d experts", NE);
    if (T < 0 || n < 0) return g53h_fail("g53h_vote: %d x %d ids", T, n);
    hipLaunchKernelGGL(k_vote, dim3(1), dim3(1024), 0, g53h_stream(), out, ids, T, n, NE);
    G53_LAUNCHED("k_vote");
    return 0;
}

extern "C" int g53h_route_decode(int *idx, float *w, int *nan_flag, int *pred, int n, const float *x, const void *gate,
                                 int gate_dt, const float *bias, const void *next_gate, int next_dt,
                                 const float *next_bias, int NE, int E, int K, int norm_topk, float routed_scale,
                                 int mb_slot, unsigned seq, size_t mb_off)
{
    if (g53h_ready()) return -1;
    if (NE < 1 || NE > 1024) return g53h_fail("g53h_route_decode: %d experts (max 1024)", NE);
    if (K < 1 || K > NE || K > GLM53F_MAX_TOPK_DEV) return g53h_fail("g53h_route_decode: topk %d", K);
    const int pn = next_gate && n > 0;
    if (pn && n > NE) return g53h_fail("g53h_route_decode: %d of %d experts", n, NE);
    if (!pn) n = 0;
    if (mb_slot >= 0 && (mb_slot >= G53H_MBOX_SLOTS || mb_off % 4 || mb_off < G53H_MBOX_SLOTS * 4 ||
                         mb_off + 4 * (size_t)(K + 1 + n) > G53H_MBOX_BYTES))
        return g53h_fail("g53h_route_decode: mailbox slot %d offset %zu", mb_slot, mb_off);
    float *ws = (float *)g53h_workspace((size_t)4 * NE * sizeof(float));
    if (!ws) return -1;
    float *sc0 = ws, *ch0 = ws + NE, *sc1 = ws + 2 * NE, *ch1 = ws + 3 * NE;
    hipLaunchKernelGGL(k_router_scores2, dim3(NE, pn ? 2 : 1), dim3(64), 0, g53h_stream(), sc0, ch0, gate, gate_dt,
                       bias, sc1, ch1, pn ? next_gate : gate, next_dt, pn ? next_bias : bias, x, NE, E);
    G53_LAUNCHED("k_router_scores2");
    unsigned *mb = mb_slot >= 0 ? g53h_mailbox_dev() : nullptr;
    const int off_w = (int)(mb_off / 4);
    if (NE <= 320)
        hipLaunchKernelGGL(k_route_decode<5>, dim3(1), dim3(128), 0, g53h_stream(), idx, w, nan_flag, sc0, ch0, bias,
                           NE, K, norm_topk, routed_scale, pred, n, sc1, ch1, mb, mb_slot, off_w, seq);
    else
        hipLaunchKernelGGL(k_route_decode<16>, dim3(1), dim3(128), 0, g53h_stream(), idx, w, nan_flag, sc0, ch0, bias,
                           NE, K, norm_topk, routed_scale, pred, n, sc1, ch1, mb, mb_slot, off_w, seq);
    G53_LAUNCHED("k_route_decode");
    if (mb) g53h_note_publish(mb_slot, seq);
    return 0;
}

/* ------------------------------------------------- speculative decode: next scores, publish ---- */
static float *g_next = nullptr;          /* [2][1024]: choice (score + bias), then score */
static G53NextReq g_next_req;

float *g53h_next_buf(void)
{
    if (!g_next) g_next = (float *)g53h_alloc(2 * 1024 * sizeof(float));
    return g_next;
}
G53NextReq *g53h_next_req(void) { return &g_next_req; }


extern "C" int g53h_decode_next(const float *x, const void *next_gate, int next_dt, const float *next_bias, int NE,
                                int E)
{
    if (g53h_ready()) return -1;
    if (NE < 1 || NE > 1024 || !x || !next_gate || !next_bias)
        return g53h_fail("g53h_decode_next: %d experts (max 1024)", NE);
    if (!g53h_next_buf()) return -1;
    g_next_req = G53NextReq{1, x, next_gate, next_dt, next_bias, NE, E};
    return 0;
}

extern "C" int g53h_route_next(const float *x, const void *next_gate, int next_dt, const float *next_bias, int NE,
                               int E)
{
    if (g53h_ready()) return -1;
    if (NE < 1 || NE > 1024) return g53h_fail("g53h_route_next: %d experts (max 1024)", NE);
    if (!g53h_next_buf()) return -1;
    hipLaunchKernelGGL(k_router_scores, dim3(NE, 1), dim3(64), 0, g53h_stream(), g_next + 1024, g_next, x, 1,
                       next_gate, next_dt, next_bias, NE, E);
    G53_LAUNCHED("k_router_scores");
    return 0;
}

/* Wave 0 takes the next layer's top-n (the selection of k_route_decode, src/core/glm53f_ops.c:
 * 1021-1042), then the workgroup writes the host's copy: idx [K], the NaN flag, pred [n] at
 * route_off_w; the error words and the output at out_off_w; then the sequence word. */
__global__ void __launch_bounds__(256) k_dec_publish(unsigned *__restrict__ mb, int slot, unsigned seq,
                                                     int route_off_w, const int *__restrict__ idx, int K,
                                                     int *__restrict__ pred, int n, const float *__restrict__ choice,
                                                     const float *__restrict__ score, int NE, int out_off_w,
                                                     const uint32_t *__restrict__ out, int nw,
                                                     const int *__restrict__ errs)
{
    /* wave 0 the top-n while the other waves copy the error words and the output */
    if (threadIdx.x < 64) {
        if (n > 0) g53_topn_token(0, (int)threadIdx.x, pred, n, choice, NE, score, nullptr);
    } else {
        uint32_t *d = mb + out_off_w;
        for (int i = threadIdx.x - 64; i < G53H_NERR; i += 192) d[i] = (uint32_t)errs[i];
        g53_copy_words(d + G53H_NERR, out, nw, (int)threadIdx.x - 64, 192);
    }
    __threadfence_block();
    __syncthreads();
    unsigned *r = mb + route_off_w;
    const int nan = ((errs[0] | errs[1]) & 2) ? 1 : 0;
    for (int i = threadIdx.x; i < K + 1 + n; i += 256)
        r[i] = (unsigned)(i < K ? idx[i] : i == K ? nan : pred[i - K - 1]);
    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(mb + slot, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

/* The mailbox areas of a publication: in range, word-aligned, not overlapping. */
static int pub_areas_bad(int slot, size_t route_off, int K, int n, size_t out_off, size_t out_bytes)
{
    return slot < 0 || slot >= G53H_MBOX_SLOTS || route_off % 4 || out_off % 4 || out_bytes % 4 ||
           route_off < G53H_MBOX_SLOTS * 4 || out_off < G53H_MBOX_SLOTS * 4 ||
           route_off + 4 * (size_t)(K + 1 + n) > G53H_MBOX_BYTES || out_off + 4 * G53H_NERR + out_bytes > G53H_MBOX_BYTES ||
           (route_off < out_off + 4 * G53H_NERR + out_bytes && out_off < route_off + 4 * (size_t)(K + 1 + n));
}

extern "C" int g53h_decode_publish(int slot, unsigned seq, size_t route_off, const int *idx_d, int K, int *pred_d,
                                   int n, int NE, size_t out_off, const void *out_d, size_t out_bytes)
{
    if (g53h_ready()) return -1;
    if (K < 1 || K > GLM53F_MAX_TOPK_DEV || n < 0 || n > NE || NE < 1 || NE > 1024 || (n > 0 && (!g_next || !pred_d)))
        return g53h_fail("g53h_decode_publish: topk %d, n %d of %d experts (g53h_route_next first)", K, n, NE);
    if (g_next_req.armed) {          /* requested, and no decode launch computed them */
        g_next_req.armed = 0;
        if (g_next_req.NE != NE ||
            g53h_route_next(g_next_req.x, g_next_req.gate, g_next_req.dt, g_next_req.bias, g_next_req.NE, g_next_req.E))
            return g53h_fail("g53h_decode_publish: the next layer's scores (%d experts) cannot be computed", NE);
    }
    if (pub_areas_bad(slot, route_off, K, n, out_off, out_bytes))
        return g53h_fail("g53h_decode_publish: slot %d, routing at %zu, %zu bytes at %zu", slot, route_off, out_bytes,
                         out_off);
    hipLaunchKernelGGL(k_dec_publish, dim3(1), dim3(256), 0, g53h_stream(), g53h_mailbox_dev(), slot, seq,
                       (int)(route_off / 4), idx_d, K, pred_d, n, g_next, g_next + 1024, NE, (int)(out_off / 4),
                       (const uint32_t *)out_d, (int)(out_bytes / 4), g53h_errblock());
    G53_LAUNCHED("k_dec_publish");
    g53h_note_publish(slot, seq);
    return 0;
}
