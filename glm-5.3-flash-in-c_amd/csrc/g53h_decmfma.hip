/* g53h_decmfma.hip - single-token decode of one MoE layer in one launch on the FP8 matrix cores,
 * over experts stored MFMA-tiled (k_dec_mfma; include/g53h.h, G53H_MAT_MTILED).
 *
 * Reference: src/core/glm53f_ops.c:1144-1342 (moe_chunk) at T = 1: the router of :945-976 (bit
 * for bit, the same selection code as the bit-exact kernels), the FP8 products of :185-228, the
 * SwiGLU of :486-494 and the combine of :1329-1340 (double, in slot order, then the shared
 * expert in float). The expert products are not the reference's fp32 FMA chains: they run on
 * v_mfma_scale_f32_16x16x128_f8f6f4 with fp32 accumulation, within the tolerance the path
 * allows (2e-3 relative / 1e-2 absolute). The bit-exact kernel (k_dec_tiled) needs one fp32
 * FMA and half a conversion per code byte on the vector ALUs; that work, not HBM, bounds it.
 * Here the vector ALUs only scale each 128-column block's sum.
 *
 * Operands. One matrix-core instruction multiplies a 16-row x 128-column tile of codes (A; lane
 * l holds row l % 16, columns 32 (l / 16) .. + 31) by a 128 x 16 operand B whose columns 0, 1
 * and 2 are the vector as three E4M3 planes (lane l: column l % 16, the same 32 columns):
 * v = 2^-k (q0 + q1 / 16 + q2 / 256), with its own k per 128-column block, passed as the
 * instruction's E8M0 scale of B together with the 16^-p of plane p. Columns 3 .. 15 are zero.
 * Column p of the result is then plane p's part of the 16 row sums of the block, already in
 * real units; each lane scales its four by the 128 x 128 block scale and accumulates them in
 * fp32. At the end the three planes' sums are added (lanes 16 g, 16 g + 1, 16 g + 2). For
 * bf16-valued inputs two planes hold v exactly; the SwiGLU activations keep about 12
 * significant bits.
 *
 * Tasks (one wave streams 32 KB, 16 KB in flight):
 *   G  rows og*8 .. og*8+7 of one slot's gate AND up matrices (A rows 0-7 gate, 8-15 up: each
 *      lane loads from its own matrix), over one half of the 32 column blocks. The two halves
 *      meet in LDS; the second to finish adds them (first half first), forms the SwiGLU and
 *      publishes the octet's 8 activations;
 *   D  16 down rows (two row octets) of one slot over its 16 column blocks, all loads in flight
 *      before the task waits for the slot's activations, which it turns into planes in its
 *      wave's LDS.
 * The work split across workgroups, the task order, the routing and the cross-workgroup
 * exchange (epoch-tagged words) are those of k_dec_tiled (g53h_dectile.hip). */
#include <hip/hip_runtime.h>
#include <math.h>

#include "g53h.h"
#include "g53h_core.h"
#include "g53h_gemv.h"
#include "g53h_kern.h"
#include "g53h_runtime.h"
#include "g53h_xwg.h"

#define G53_DM_NW 8                 /* waves per workgroup                                */
#ifndef G53_DM_P
#define G53_DM_P 16                 /* G tasks: 1 KB half-tiles in flight per wave        */
#endif
#define G53_DM_NT (64 * G53_DM_NW)
#define G53_DM_BB 512               /* LDS bytes of one block's B operand (4 groups x 4 x 32) */
#define G53_DM_NGO (G53_DEC_I / 8)
#define G53_DM_NDO (G53_DEC_E / 8)
#define G53_DM_MAXGO 2
#define G53_DM_MAXDO 4
#define G53_DM_DTAB 24576
#define G53_DM_ROT 16
#ifndef G53_DM_BPIPE
#define G53_DM_BPIPE 1              /* B operands read by every lane, one block ahead          */
#endif
#ifndef G53_DM_RING1
#define G53_DM_RING1 1              /* G tasks: PB + 1 register slots, requests one block early */
#endif
#ifndef G53_DM_PIN
#define G53_DM_PIN 2                /* blocks between two pins of the block arithmetic     */
#endif
#ifndef G53_DM_NPX
#define G53_DM_NPX 3                /* E4M3 planes of x                                   */
#endif
#ifndef G53_DM_NPA
#define G53_DM_NPA 3                /* E4M3 planes of the SwiGLU activations              */
#endif
#define G53_DM_LD(p) __builtin_nontemporal_load(p)

typedef int g53_m8i __attribute__((ext_vector_type(8)));
typedef float g53_m4f __attribute__((ext_vector_type(4)));
typedef int g53_v4i_dm __attribute__((ext_vector_type(4)));
#if defined(__HIP_DEVICE_COMPILE__)
typedef __attribute__((address_space(1))) const g53_u4 g53_mgv4;
#else
typedef const g53_u4 g53_mgv4;
#endif
#if defined(__HIP_DEVICE_COMPILE__)
typedef __attribute__((address_space(1))) const float4 g53_mgf4;
#else
typedef const float4 g53_mgf4;
#endif

struct G53MfmaArgs {
    float *out;
    const float *x;
    const uint16_t *router;
    const float *bias;
    const G53hExpert *experts;
    const G53hExpert *shared;
    g53_u64 *score;
    g53_u64 *act;
    int *err;
    int *idx_out;
    float *w_out;
    const int *idx_in;
    const float *w_in;
    int NE, K, norm_topk;
    unsigned epoch;
    float routed_scale, limit;
    int spin;
    g53_u64 *trace;
    const uint16_t *nrouter;       /* optional: the next layer's bf16 router [NE][E] and bias, */
    const float *nbias;            /* whose scores (choice = score + bias) spare waves write */
    float *nscore, *nchoice;       /* to nscore / nchoice [NE] (the prediction's input)      */
};

__device__ __forceinline__ bool g53_desc_mtiled(const G53hExpert &e)
{
    return g53_desc_ok(e) && (e.gate.flags & G53H_MAT_MTILED) && (e.up.flags & G53H_MAT_MTILED) &&
           (e.down.flags & G53H_MAT_MTILED);
}

/* NV consecutive values of a 128-column block as B-operand bytes; the block's 128 / NV lanes
 * (a quad for NV = 32, eight lanes for NV = 16, consecutive) call this together. Three E4M3
 * planes of 2^k v (NV bytes each) go to dst + 32 p, zeros to dst + 96 (the columns past the
 * planes read them), dst being this lane's place in its 32-value group. A lane that starts a
 * group (first) also writes the E8M0 scale bytes of the 16 lanes that read the group at sc:
 * 127 - k - 4 p for column p < 3. k = 8 - exponent(max |v| over the block), so that 2^k |v| <
 * 256, clamped to [-100, 100] (blocks below 2^-92 in magnitude then round to zero). One k for
 * the block: the matrix core takes one B scale per 32 values of a column, from lanes that do
 * not follow the operand's lane order, so all four of a column agree. */
template <int NV, int NP = 3>
__device__ __forceinline__ void g53_dm_planes(const float (&v)[NV], uint8_t *dst, uint8_t *sc, bool first)
{
    static_assert(NV == 16 || NV == 32, "a half or a whole group per lane");
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) m = fmaxf(m, fabsf(v[i]));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0xB1, 0xf, 0xf, true)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0x4E, 0xf, 0xf, true)));
    if (NV == 16) m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0x141, 0xf, 0xf, true)));
    int ex = 0;
    if (m > 0.0f && m <= 3.0e38f) (void)frexpf(m, &ex);
    const int k = min(100, max(-100, 8 - ex));
    const float s = ldexpf(1.0f, k);
    uint32_t q[3][NV / 4];
#pragma unroll
    for (int w = 0; w < NV / 4; w++) {
        float r[4] = {v[4 * w] * s, v[4 * w + 1] * s, v[4 * w + 2] * s, v[4 * w + 3] * s};
#pragma unroll
        for (int p = 0; p < 3; p++) {
            int c = __builtin_amdgcn_cvt_pk_fp8_f32(r[0], r[1], 0, false);
            c = __builtin_amdgcn_cvt_pk_fp8_f32(r[2], r[3], c, true);
            q[p][w] = p < NP ? (uint32_t)c : 0u;
            if (p < 2) {
                r[0] = (r[0] - __builtin_amdgcn_cvt_f32_fp8(c, 0)) * 16.0f;
                r[1] = (r[1] - __builtin_amdgcn_cvt_f32_fp8(c, 1)) * 16.0f;
                r[2] = (r[2] - __builtin_amdgcn_cvt_f32_fp8(c, 2)) * 16.0f;
                r[3] = (r[3] - __builtin_amdgcn_cvt_f32_fp8(c, 3)) * 16.0f;
            }
        }
    }
#pragma unroll
    for (int p = 0; p < 3; p++)
#pragma unroll
        for (int h = 0; h < NV / 16; h++)
            ((uint4 *)(dst + 32 * p))[h] = make_uint4(q[p][4 * h], q[p][4 * h + 1], q[p][4 * h + 2], q[p][4 * h + 3]);
#pragma unroll
    for (int h = 0; h < NV / 16; h++) ((uint4 *)(dst + 96))[h] = make_uint4(0u, 0u, 0u, 0u);
    if (first) {
        const uint32_t b0 = (uint32_t)(127 - k), b1 = b0 - 4, b2 = b0 - 8;
        const uint32_t w0 = b0 | (b1 << 8) | (b2 << 16) | (127u << 24), wr = 0x7f7f7f7fu;
        *(uint4 *)sc = make_uint4(w0, wr, wr, wr);
    }
}

/* A lane's 32 bytes of one block: its 16 bytes of each 1 KB half-tile (q points at the first;
 * the second follows 512 bytes on), as one 8-register operand. */
__device__ __forceinline__ g53_m8i g53_dm_ld(g53_mgv4 *q)
{
    const g53_u4 h0 = G53_DM_LD(q), h1 = G53_DM_LD(q + 32);
    return __builtin_shufflevector(__builtin_bit_cast(g53_v4i_dm, h0), __builtin_bit_cast(g53_v4i_dm, h1), 0, 1, 2,
                                   3, 4, 5, 6, 7);
}

/* One block on the matrix cores: A (the lane's 32 code bytes), B and its scale from LDS; the
 * result times the lane's block scale s added to acc. */
__device__ __forceinline__ void g53_dm_block(g53_m4f &acc, const g53_m8i &a, const uint8_t *bq, const uint8_t *bs,
                                             bool bl, float s)
{
    /* only the lanes of columns 0-2 hold planes: the others pass zeros without reading LDS */
    g53_m8i b = {0, 0, 0, 0, 0, 0, 0, 0};
    int bscale = 127;
    if (bl) {
        b = *(const g53_m8i *)bq;
        bscale = *bs;
    }
    g53_m4f c = {0.0f, 0.0f, 0.0f, 0.0f};
    c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, bscale);
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = __builtin_fmaf(c[i], s, acc[i]);
}

/* The same with B and its scale already in registers (read a block ahead by every lane: the
 * lanes of columns 3-15 read the zero slot of their group and the scale 0x7f). */
__device__ __forceinline__ void g53_dm_mma(g53_m4f &acc, const g53_m8i &a, const g53_m8i &b, int bscale, float s)
{
    g53_m4f c = {0.0f, 0.0f, 0.0f, 0.0f};
    c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, bscale);
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = __builtin_fmaf(c[i], s, acc[i]);
}

/* The sums of the three planes into the lanes of column 0 (lanes 16 g): rows 4 g .. 4 g + 3. */
__device__ __forceinline__ g53_m4f g53_dm_planesum(const g53_m4f &acc)
{
    g53_m4f r;
#pragma unroll
    for (int i = 0; i < 4; i++) r[i] = (acc[i] + __shfl_down(acc[i], 1)) + __shfl_down(acc[i], 2);
    return r;
}

/* ------------------------------------------------ int4 experts (FP4 matrix cores) ---- */
/* A routed expert in the int4 MFMA-tiled layout (include/g53h.h, G53H_MAT_I4 | G53H_MAT_MTILED)
 * with the released shapes and one step per row and 64 columns. */
__device__ __forceinline__ bool g53_desc_i4m(const G53hExpert &e)
{
    const G53hMat *mm[3] = {&e.gate, &e.up, &e.down};
    const int rows[3] = {G53_DEC_I, G53_DEC_I, G53_DEC_E}, cols[3] = {G53_DEC_E, G53_DEC_E, G53_DEC_I};
    bool ok = true;
    for (int i = 0; i < 3; i++)
        ok = ok && mm[i]->w && mm[i]->s && (mm[i]->flags & G53H_MAT_I4) && (mm[i]->flags & G53H_MAT_MTILED) &&
             mm[i]->rows == rows[i] && mm[i]->cols == cols[i] && mm[i]->bc == 64 && mm[i]->scols == cols[i] / 64;
    return ok;
}

/* The int4 products of one block. Level l = 4 h + b (h, b < 4) minus 8: the A operand is FP4
 * (E2M1), whose codes 0-3 are the values 0, 0.5, 1, 1.5, so the two-bit fields h and b of the
 * lane's 32 levels are two FP4 planes as they lie ((r >> 2) & 0x3.., r & 0x3..), taken at A
 * scales 2^3 (4 h) and 2^1 (b); a third product with every code -4 (0xE) at scale 2^1 adds
 * -8 times the block's inputs. The matrix core reads lane l's 32 FP4 values as row l % 16 and
 * columns (of B's order) 64 (g & 1) + 16 (g >> 1) + 0..15 and + 32 .. + 47 (g = l / 16), which
 * is where the MFMA-tiled layout puts them. B: column m < 6 of K-group g carries plane m - 3 (g
 * >> 1) of x over the block's 64-column half g >> 1 (zeros elsewhere), so that result column m
 * is one plane of one half; each lane scales its four rows by their half's steps (st). */
__device__ __forceinline__ void g53_dm_i4_mma(g53_m4f &acc, const g53_u4 &r, const g53_m8i &b, int bscale,
                                              const float4 &st)
{
    const g53_m8i ah = {(int)((r.x >> 2) & 0x33333333u), (int)((r.y >> 2) & 0x33333333u),
                        (int)((r.z >> 2) & 0x33333333u), (int)((r.w >> 2) & 0x33333333u), 0, 0, 0, 0};
    const g53_m8i ab = {(int)(r.x & 0x33333333u), (int)(r.y & 0x33333333u), (int)(r.z & 0x33333333u),
                        (int)(r.w & 0x33333333u), 0, 0, 0, 0};
    const g53_m8i ac = {(int)0xEEEEEEEEu, (int)0xEEEEEEEEu, (int)0xEEEEEEEEu, (int)0xEEEEEEEEu, 0, 0, 0, 0};
    g53_m4f c = {0.0f, 0.0f, 0.0f, 0.0f};
    c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ah, b, c, 4, 0, 0, 130, 0, bscale);
    c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ab, b, c, 4, 0, 0, 128, 0, bscale);
    c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ac, b, c, 4, 0, 0, 128, 0, bscale);
    acc[0] = __builtin_fmaf(c[0], st.x, acc[0]);
    acc[1] = __builtin_fmaf(c[1], st.y, acc[1]);
    acc[2] = __builtin_fmaf(c[2], st.z, acc[2]);
    acc[3] = __builtin_fmaf(c[3], st.w, acc[3]);
}

/* This lane's B slot in a K-group's 128 LDS bytes (plane 0-2, or 3: the zeros) and its scale
 * byte (the plane's, the same in all four K-groups of the column; 3: the unit scale). */
__device__ __forceinline__ int g53_dm_i4_slot(int m, int grp)
{
    const int p = m - 3 * (grp >> 1);
    return (unsigned)p < 3u ? p : 3;
}
__device__ __forceinline__ int g53_dm_i4_sc(int m) { return m < 6 ? m % 3 : 3; }

/* The sums of the six columns into the lanes of column 0 (lanes 16 g): rows 4 g .. 4 g + 3. */
__device__ __forceinline__ g53_m4f g53_dm_i4_colsum(const g53_m4f &acc)
{
    g53_m4f r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float t = (acc[i] + __shfl_down(acc[i], 1)) + __shfl_down(acc[i], 2);
        r[i] = t + __shfl_down(t, 3);
    }
    return r;
}

__device__ __forceinline__ const uint8_t *g53_dm_uptr(const uint8_t *p)
{
    const g53_u64 v = (g53_u64)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const uint8_t *)(uintptr_t)(((g53_u64)hi << 32) | lo);
}

#define G53_MTRACE(k) do { if (a.trace && lane == 0) \
    a.trace[(size_t)blockIdx.x * 192 + (k)] = __builtin_amdgcn_s_memrealtime(); } while (0)

/* I4: the routed experts are int4, int4 MFMA-tiled (G53H_MAT_I4 | G53H_MAT_MTILED; the reference's
 * --experts int4), multiplied on the FP4 matrix cores (g53_dm_i4_mma); the shared expert stays
 * FP8 MFMA-tiled. */
template <bool I4>
__global__ void __launch_bounds__(G53_DM_NT, 1) k_dec_mfma(G53MfmaArgs a)
{
    __shared__ __attribute__((aligned(16))) uint8_t xq[G53_DEC_NBE * G53_DM_BB];      /* x, B operand    */
    __shared__ __attribute__((aligned(16))) uint8_t xsc[G53_DEC_NBE * 64];           /* its scales      */
    __shared__ __attribute__((aligned(16))) uint8_t aq[G53_DM_NW][G53_DEC_NBI / 2 * G53_DM_BB];
    __shared__ __attribute__((aligned(16))) uint8_t asc[G53_DM_NW][G53_DEC_NBI / 2 * 64];
    __shared__ float dpart[G53_DM_MAXDO / 2][2][16][G53_DEC_MAXK + 1];   /* D half sums          */
    __shared__ int dcnt[G53_DM_MAXDO / 2][G53_DEC_MAXK + 1];
    __shared__ __attribute__((aligned(16))) uint2 dtab[G53_DM_DTAB / 8];
    __shared__ G53hExpert st[G53_DEC_MAXK + 1];
    __shared__ float biasl[G53_DEC_MAXNE];
    __shared__ float cvals[G53_DM_MAXDO * 8][G53_DEC_MAXK + 1];
    __shared__ float gup[G53_DEC_MAXK + 1][G53_DM_MAXGO][2][16];   /* half sums, gate 0-7, up 8-15 */
    __shared__ int gucnt[G53_DEC_MAXK + 1][G53_DM_MAXGO];
    __shared__ float sw[64];
    __shared__ int sidx[16], ebuf[64];
    __shared__ uint32_t kbuf[64];
    __shared__ uint64_t etab[32];
    __shared__ int qctr, ndone, routed, nrouted, inited, xready, sready;

    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int m = lane & 15, grp = lane >> 4;
    const int K = a.K, hs = a.shared ? 1 : 0;
    const int G = gridDim.x, b = blockIdx.x;
    const int go_lo = G53_DM_NGO * b / G, n_go = G53_DM_NGO * (b + 1) / G - go_lo;
    const int do_lo = G53_DM_NDO * b / G, n_do = G53_DM_NDO * (b + 1) / G - do_lo;
    const int ng = 2 * n_go, nd = 2 * ((n_do + 1) >> 1), nslot = hs + K;
    const int nR = a.idx_in ? 0 : (a.NE > b ? (a.NE - 1 - b) / G + 1 : 0);
    const int nN = a.nrouter ? (a.NE > b ? (a.NE - 1 - b) / G + 1 : 0) : 0;   /* next-layer rows */
    const int words = (int)(sizeof(G53hExpert) / 4);
    const bool dstage = a.NE * (int)sizeof(G53hExpert) <= G53_DM_DTAB;
    const int n_setup = G53_DM_NW - 1 - nR - nN;

    G53_MTRACE(0);
    if (threadIdx.x == 0) { qctr = 0; ndone = 0; routed = 0; nrouted = 0; inited = 0; xready = 0; sready = 0; }
    __syncthreads();
    if (w < nR || w == G53_DM_NW - 1) __builtin_amdgcn_s_setprio(3);
    if (w < nR) {
        /* router row b + w G (x read straight from memory), published at once */
        g53_u4 cr[8];
        g53_mgv4 *q = (g53_mgv4 *)(a.router + (size_t)(b + w * G) * G53_DEC_E + lane * 64);
#pragma unroll
        for (int k = 0; k < 8; k++) cr[k] = q[k];
        const double d = g53_router_row(cr, a.x, lane);
        if (lane == 0) g53_st_tag(a.score + b + w * G, g53_tag(a.epoch, g53_sigmoidf_tab((float)d, g53_exp2_tab_dev)));
        if (w == 0) G53_MTRACE(2);
        __builtin_amdgcn_s_setprio(0);
    } else if (w < nR + nN) {
        /* the next layer's router row b + (w - nR) G on the same x: its score and choice for the
         * prediction (the arithmetic of k_router_scores, bit for bit) */
        const int e = b + (w - nR) * G;
        g53_u4 cr[8];
        g53_mgv4 *q = (g53_mgv4 *)(a.nrouter + (size_t)e * G53_DEC_E + lane * 64);
#pragma unroll
        for (int k = 0; k < 8; k++) cr[k] = q[k];
        const double d = g53_router_row(cr, a.x, lane);
        if (lane == 0) {
            const float sc = g53_sigmoidf_tab((float)d, g53_exp2_tab_dev);
            a.nscore[e] = sc;
            a.nchoice[e] = sc + a.nbias[e];
        }
    } else if (w < G53_DM_NW - 1) {
        /* the set-up: x as B-operand planes (thread t: group t of 32 values), the expert table,
         * the shared descriptor, the exponential's table */
        const int ti = threadIdx.x - 64 * (nR + nN), nt = (G53_DM_NW - 1 - nR - nN) * 64;
        /* the shared descriptor first: the first tasks (the shared expert's) need it to issue
         * their code loads, and may start as soon as it is in LDS */
        int dw = 0;
        if (ti < words && hs) dw = ((const int *)a.shared)[ti];
        if (ti < words) ((int *)&st[K])[ti] = dw;
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        G53_CBAR();
        if (lane == 0) g53_lds_add(&sready, 1);
        float v[16];
        const bool xg = ti < G53_DEC_E / 16;                       /* 256 half-groups, nt >= 256 */
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float4 f = xg ? ((const float4 *)a.x)[ti * 4 + k] : make_float4(0.f, 0.f, 0.f, 0.f);
            v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
        }
        const uint64_t et = ti < 32 ? g53_exp2_tab_dev[ti] : 0;
        /* the expert table's loads go out with the others, in one round */
        constexpr int DPER = 16;
        const int n8 = dstage ? a.NE * (int)(sizeof(G53hExpert) / 8) : 0;
        const uint2 *t8 = (const uint2 *)a.experts;
        uint2 dv[DPER];
#pragma unroll
        for (int k = 0; k < DPER; k++) dv[k] = ti + k * nt < n8 ? t8[ti + k * nt] : make_uint2(0u, 0u);
        /* what the tasks' arithmetic needs: x as planes, the SwiGLU's table and counters */
        if (ti < (G53_DEC_MAXK + 1) * G53_DM_MAXGO) (&gucnt[0][0])[ti] = 0;
        if (ti < (G53_DEC_MAXK + 1) * (G53_DM_MAXDO / 2)) (&dcnt[0][0])[ti] = 0;
        if (ti < 32) etab[ti] = et;
        if (xg) {                 /* thread t: values 16 t .. 16 t + 15 (block t / 8, group t / 2 % 4) */
            const int kb = ti >> 3, g = (ti >> 1) & 3, hf = ti & 1;
            g53_dm_planes<16, G53_DM_NPX>(v, xq + kb * G53_DM_BB + g * 128 + 16 * hf, xsc + kb * 64 + g * 16, hf == 0);
        }
        /* fewer than 256 set-up threads (layers of more than 768 experts): the rest, a whole
         * wave at a time (nt is a multiple of 64, so the eight lanes of a block stay together) */
        for (int t = ti + nt; t < G53_DEC_E / 16; t += nt) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float4 f = ((const float4 *)a.x)[t * 4 + k];
                v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
            }
            const int kb = t >> 3, g = (t >> 1) & 3, hf = t & 1;
            g53_dm_planes<16, G53_DM_NPX>(v, xq + kb * G53_DM_BB + g * 128 + 16 * hf, xsc + kb * 64 + g * 16, hf == 0);
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        G53_CBAR();
        if (lane == 0) g53_lds_add(&xready, 1);
        G53_MTRACE(144 + w);
        if (w == G53_DM_NW - 2) G53_MTRACE(15);
        /* the expert table, which only the routed tasks read (after the routing) */
#pragma unroll
        for (int k = 0; k < DPER; k++)
            if (ti + k * nt < n8) dtab[ti + k * nt] = dv[k];
        for (int q = ti + DPER * nt; q < n8; q += nt) dtab[q] = t8[q];
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        G53_CBAR();
        if (lane == 0) g53_lds_add(&inited, 1);
        G53_MTRACE(160 + w);
    }
    if (w != G53_DM_NW - 1 && !g53_wait_lds(&sready, n_setup) && lane == 0) g53_flag_err(a.err, 1);

    /* the routing: top-k, weights (reference :945-976), bit for bit */
    if (w == G53_DM_NW - 1) {

        g53_u64 t_seen = 0, t_tau = 0, t_rank = 0;
        int n_polls = 0;
        bool ok = true;
        if (a.idx_in) {
            if (lane < K) { sidx[lane] = a.idx_in[lane]; sw[lane] = a.w_in[lane]; }
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();
        } else if (a.NE <= 64 * 5)
            ok = g53_route_wave<5>(a.score, biasl, a.NE, K, a.norm_topk, a.routed_scale, a.epoch, sidx, sw, kbuf, ebuf,
                                   a.err, lane, t_seen, n_polls, t_tau, t_rank, a.spin, &nrouted, nullptr, a.bias);
        else
            ok = g53_route_wave<G53_DEC_MAXNE / 64>(a.score, biasl, a.NE, K, a.norm_topk, a.routed_scale, a.epoch,
                                                    sidx, sw, kbuf, ebuf, a.err, lane, t_seen, n_polls, t_tau, t_rank,
                                                    a.spin, &nrouted, nullptr, a.bias);
        if (!ok) {
            if (lane == 0) g53_flag_err(a.err, 1);
            if (lane < K) { sidx[lane] = -1; sw[lane] = 0.0f; }
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();
        }
        /* every slot handed over (given routing, missing scores, fewer selectable experts) */
        G53_CBAR();
        if (lane == 0) {
            const int have = g53_lds_ld(&nrouted);
            if (have < K) (void)g53_lds_add(&nrouted, K - have);
        }
        G53_CBAR();
        if (lane == 0) g53_lds_add(&routed, 1);
        __builtin_amdgcn_s_setprio(0);
        if (b == 0 && lane < K && !a.idx_in) {
            if (a.idx_out) a.idx_out[lane] = sidx[lane];
            if (a.w_out) a.w_out[lane] = sw[lane];
        }
        G53_MTRACE(1);
        if (a.trace && lane == 0) {
            a.trace[(size_t)blockIdx.x * 192 + 12] = t_seen;
            a.trace[(size_t)blockIdx.x * 192 + 13] = t_tau;
            a.trace[(size_t)blockIdx.x * 192 + 14] = t_rank;
        }
    }
    const bool shared_ok = hs && st[K].gate.w && g53_desc_mtiled(st[K]);
    if (hs && st[K].gate.w && !shared_ok && b == 0 && threadIdx.x == 0) g53_flag_err(a.err, 8);
    const int n_task = nslot * (ng + nd), n_dall = nslot * (nd >> 1);
    uint8_t *myaq = aq[w], *myasc = asc[w];
    bool staged = false, xr = false;
    G53_MTRACE(128 + w);
    for (;;) {
        int t = 0;
        if (lane == 0) t = g53_lds_add(&qctr, 1);
        t = __builtin_amdgcn_readfirstlane(t);
        if (t >= n_task) break;
        if (t < 32) G53_MTRACE(64 + 2 * t);
        int s, idx;
        bool is_g;
        if (!a.idx_in) {
            /* routed here: the shared expert's G and D tasks fill the routing's wait */
            const int i_sd = hs * ng, i_rg = i_sd + hs * nd, i_rd = i_rg + K * ng;
            if (t < i_sd) { s = K; is_g = true; idx = t; }
            else if (t < i_rg) { s = K; is_g = false; idx = t - i_sd; }
            else if (t < i_rd) { s = (t - i_rg) / ng; is_g = true; idx = (t - i_rg) - s * ng; }
            else { s = (t - i_rd) / nd; is_g = false; idx = (t - i_rd) - s * nd; }
        } else {
            /* routing given: no wait to fill, so the shared expert's D task comes after every G
             * task, when its activations are long complete */
            const int j_rg = hs * ng, j_sd = j_rg + K * ng, j_rd = j_sd + hs * nd;
            if (t < j_rg) { s = K; is_g = true; idx = t; }
            else if (t < j_sd) { s = (t - j_rg) / ng; is_g = true; idx = (t - j_rg) - s * ng; }
            else if (t < j_rd) { s = K; is_g = false; idx = t - j_sd; }
            else { s = (t - j_rd) / nd; is_g = false; idx = (t - j_rd) - s * nd; }
        }
        if (s < K && g53_lds_ld(&nrouted) <= s) {          /* slot s is chosen: its index is in */
            if (!g53_wait_lds(&nrouted, s + 1) && lane == 0) g53_flag_err(a.err, 1);
        }
        if (s < K && !staged) {                  /* the staged expert table (long complete by now) */
            if (!g53_wait_lds(&inited, n_setup) && lane == 0) g53_flag_err(a.err, 1);
            staged = true;
        }
        G53hExpert ex;
        bool usable;
        if (s == K) {
            ex = st[K];
            usable = shared_ok;
        } else {
            const int e = sidx[s];
            if (e >= 0 && e < a.NE) ex = dstage ? ((const G53hExpert *)dtab)[e] : a.experts[e];
            else ex.gate.w = nullptr;
            usable = ex.gate.w != nullptr && (I4 ? g53_desc_i4m(ex) : g53_desc_mtiled(ex));
            if (ex.gate.w && !usable && lane == 0) g53_flag_err(a.err, 8);
        }
        const bool present = __builtin_amdgcn_readfirstlane((int)usable) != 0;
        if (is_g) {
            if (!present) continue;                   /* its activations are never read */
            const int ogl = idx >> 1, og = go_lo + ogl, h = idx & 1;
            g53_m4f vg;
            if (I4 && s < K) {
                /* int4: lane's row as for FP8; its 16 bytes of block kb at + kb * 512, its four
                 * rows' steps of the half of its column (float4 at + kb * 16) */
                const uint8_t *gw = g53_dm_uptr(ex.gate.w), *uw = g53_dm_uptr(ex.up.w);
                const uint8_t *wb = m < 8 ? gw : uw;
                const size_t u0 = (size_t)og * G53_DEC_NBE + 16 * h;
                const uint8_t *pl = wb + u0 * 512 + (grp * 8 + (m & 7)) * 16;
                const float *sb = (grp < 2 ? ex.gate.s : ex.up.s) + u0 * 16 + (m < 6 ? m / 3 : 0) * 8 + 4 * (grp & 1);
                __builtin_amdgcn_sched_barrier(0);
                constexpr int NB = G53_DEC_NBE / 2;
                g53_u4 r[NB];
                float4 stp[NB];
#pragma unroll
                for (int j = 0; j < NB; j++) {
                    r[j] = G53_DM_LD((g53_mgv4 *)(pl + 512 * j));
                    stp[j] = *(g53_mgf4 *)(sb + 16 * j);
                }
                if (!xr) {
                    if (!g53_wait_lds(&xready, n_setup) && lane == 0) g53_flag_err(a.err, 1);
                    xr = true;
                }
                g53_m4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
                const uint8_t *bq0 = xq + 16 * h * G53_DM_BB + grp * 128 + g53_dm_i4_slot(m, grp) * 32;
                const uint8_t *bs0 = xsc + 16 * h * 64 + grp * 16 + g53_dm_i4_sc(m);
                g53_m8i bn = *(const g53_m8i *)bq0;
                int sn = bs0[0];
#pragma unroll
                for (int kb = 0; kb < NB; kb++) {
                    const g53_m8i bc = bn;
                    const int sc = sn;
                    if (kb + 1 < NB) {
                        bn = *(const g53_m8i *)(bq0 + (kb + 1) * G53_DM_BB);
                        sn = bs0[(kb + 1) * 64];
                    }
                    g53_dm_i4_mma(acc, r[kb], bc, sc, stp[kb]);
                    if ((kb % G53_DM_PIN) == G53_DM_PIN - 1) asm volatile("" : "+v"(acc));
                }
                vg = g53_dm_i4_colsum(acc);
            } else {
            /* lane's row: gate rows for A rows 0-7, up rows for 8-15; its 16 bytes of half-tile i
             * of block kb at + kb KB + 512 i */
            const uint8_t *gw = g53_dm_uptr(ex.gate.w), *uw = g53_dm_uptr(ex.up.w);
            const uint8_t *wb = m < 8 ? gw : uw;
            const uint8_t *pl = wb + ((size_t)og * G53_DEC_NBE + 16 * h) * 1024 + (grp * 8 + (m & 7)) * 16;
            /* block scales: lane j < 16 gate's block 16 h + j, lane 16 + j up's */
            const float *sp = lane < 16 ? ex.gate.s + (size_t)(og >> 4) * ex.gate.scols + 16 * h + lane
                                        : ex.up.s + (size_t)(og >> 4) * ex.up.scols + 16 * h + (lane & 15);
            const float scv = lane < 32 ? *(const g53_gf *)sp : 0.0f;
            __builtin_amdgcn_sched_barrier(0);
            g53_mgv4 *q = (g53_mgv4 *)pl;
            constexpr int NB = G53_DEC_NBE / 2, PB = G53_DM_P / 2;
#if G53_DM_RING1
            g53_m8i r[PB + 1];
#else
            g53_m8i r[PB];
#endif
#pragma unroll
            for (int j = 0; j < PB; j++) r[j] = g53_dm_ld(q + 64 * j);
            if (!xr) {                            /* x as planes: the first multiply needs them */
                if (!g53_wait_lds(&xready, n_setup) && lane == 0) g53_flag_err(a.err, 1);
                xr = true;
            }
            g53_m4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
            const int sbits = __float_as_int(scv);
            const uint8_t *bq0 = xq + 16 * h * G53_DM_BB + grp * 128 + min(m, 3) * 32;
            const uint8_t *bs0 = xsc + 16 * h * 64 + lane;
#if G53_DM_RING1
            /* a ring of PB + 1: block kb + PB is requested before block kb is multiplied, so
             * the multiply's operand reads never delay the next request */
#if G53_DM_BPIPE
            g53_m8i bn = *(const g53_m8i *)bq0;
            int sn = bs0[0];
#endif
#pragma unroll
            for (int kb = 0; kb < NB; kb++) {
                if (kb + PB < NB) r[(kb + PB) % (PB + 1)] = g53_dm_ld(q + 64 * (kb + PB));
                const float sg = __int_as_float(__builtin_amdgcn_readlane(sbits, kb));
                const float su = __int_as_float(__builtin_amdgcn_readlane(sbits, 16 + kb));
#if G53_DM_BPIPE
                const g53_m8i bc = bn;
                const int sc = sn;
                if (kb + 1 < NB) {
                    bn = *(const g53_m8i *)(bq0 + (kb + 1) * G53_DM_BB);
                    sn = bs0[(kb + 1) * 64];
                }
                g53_dm_mma(acc, r[kb % (PB + 1)], bc, sc, grp < 2 ? sg : su);
#else
                g53_dm_block(acc, r[kb % (PB + 1)], bq0 + kb * G53_DM_BB, bs0 + kb * 64, m < 3, grp < 2 ? sg : su);
#endif
                if ((kb % G53_DM_PIN) == G53_DM_PIN - 1) asm volatile("" : "+v"(acc));
            }
#else
#pragma unroll 1
            for (int k0 = 0; k0 < NB; k0 += PB) {
#pragma unroll
                for (int j = 0; j < PB; j++) {
                    const int kb = k0 + j;
                    const float sg = __int_as_float(__builtin_amdgcn_readlane(sbits, kb));
                    const float su = __int_as_float(__builtin_amdgcn_readlane(sbits, 16 + kb));
                    /* the result's rows 0-7 (gate) sit in lanes 0-31, rows 8-15 (up) in 32-63 */
                    g53_dm_block(acc, r[j], bq0 + kb * G53_DM_BB, bs0 + kb * 64, m < 3, grp < 2 ? sg : su);
                    /* pin the arithmetic every G53_DM_PIN blocks: the compiler would otherwise
                     * hoist every block's LDS operand and sink the matrix work past the loads,
                     * keeping all operands live at once */
                    if ((j % G53_DM_PIN) == G53_DM_PIN - 1) asm volatile("" : "+v"(acc));
                    if (k0 + PB < NB) r[j] = g53_dm_ld(q + 64 * (kb + PB));
                }
            }
#endif
            vg = g53_dm_planesum(acc);
            }
            if (m == 0)
#pragma unroll
                for (int i = 0; i < 4; i++) gup[s][ogl][h][4 * grp + i] = vg[i];
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();
            G53_CBAR();
            int second = 0;
            if (lane == 0) second = g53_lds_add(&gucnt[s][ogl], 1) == 1;
            if (__builtin_amdgcn_readfirstlane(second)) {
                G53_CBAR();
                if (lane < 8) {
                    const float gs = gup[s][ogl][0][lane] + gup[s][ogl][1][lane];
                    const float us = gup[s][ogl][0][8 + lane] + gup[s][ogl][1][8 + lane];
                    const float act = g53_swiglu1_tab(gs, us, a.limit, etab);
                    g53_st_tag(a.act + (size_t)s * G53_DEC_I + og * 8 + lane, g53_tag(a.epoch, act));
                }
            }
            if (t < 32) G53_MTRACE(65 + 2 * t);
            continue;
        }
        /* D half-task: down rows of octets oa, ob over column blocks 8 hd .. 8 hd + 7 */
        const int dp = idx >> 1, hd = idx & 1;
        const int oa = do_lo + 2 * dp, ob = oa + 1 < do_lo + n_do ? oa + 1 : oa;
        /* the half's 1024 activations: lane l takes values 16 l .. 16 l + 15 of it (block
         * l / 8, group l / 2 % 4), re-read coherently until every tag is this launch's, then
         * writes them as B-operand planes into this wave's LDS */
        g53_u64 *act_s = a.act + (size_t)s * G53_DEC_I + 1024 * hd;
        const __amdgpu_buffer_rsrc_t rs = g53_rsrc(act_s);
        const int v0 = 16 * lane;
        g53_mgv4 *src = (g53_mgv4 *)(act_s + v0);
        float av[16];
        uint32_t pend = 0;
        auto load_all = [&]() {
            pend = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const g53_u4 qv = src[k];
                av[2 * k] = __uint_as_float(qv.x);
                av[2 * k + 1] = __uint_as_float(qv.z);
                if (qv.y != a.epoch) pend |= 1u << (2 * k);
                if (qv.w != a.epoch) pend |= 1u << (2 * k + 1);
            }
        };
        /* stage_act follows a load_all issued before the task's code loads: usually the slot's
         * activations are long complete and that one round trip suffices, and the loads complete
         * in order, so the activations need not wait for the codes */
        auto stage_act = [&]() {
            int spins = 0;
            if (__ballot(pend != 0)) {
                /* not yet: the last value of every row octet (2 KB per poll instead of the half's
                 * 8 KB), with a growing back-off, then the values again */
                const __amdgpu_buffer_rsrc_t rsl = rs;
                int nap = 1;
                for (;;) {
                    g53_u64 tv[2];
#pragma unroll
                    for (int k = 0; k < 2; k++) tv[k] = g53_ld_coh64(rsl, 8 * ((lane + 64 * k) * 8 + 7));
                    const int stale = ((unsigned)(tv[0] >> 32) != a.epoch) | ((unsigned)(tv[1] >> 32) != a.epoch);
                    if (!__ballot(stale)) break;
                    if (++spins > a.spin / 16 + 1) { if (lane == 0) g53_flag_err(a.err, 1); break; }
                    for (int qq = 0; qq < nap; qq++) __builtin_amdgcn_s_sleep(8);
                    if (nap < 8) nap *= 2;
                }
                load_all();
            }
            spins = 0;
            while (__ballot(pend != 0)) {
                if (++spins > a.spin) { if (lane == 0) g53_flag_err(a.err, 1); break; }
                g53_backoff();
#pragma unroll
                for (int mm = 0; mm < 16; mm++) {
                    if (!(pend & (1u << mm))) continue;
                    const g53_u64 tv = g53_ld_coh64(rs, 8 * (v0 + mm));
                    if ((unsigned)(tv >> 32) == a.epoch) {
                        av[mm] = __uint_as_float((uint32_t)tv);
                        act_s[v0 + mm] = tv;
                        pend &= ~(1u << mm);
                    }
                }
            }
            const int kb = lane >> 3, g = (lane >> 1) & 3, hf = lane & 1;
            g53_dm_planes<16, G53_DM_NPA>(av, myaq + kb * G53_DM_BB + g * 128 + 16 * hf, myasc + kb * 64 + g * 16,
                                          hf == 0);
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();
        };
        g53_m4f v = {0.0f, 0.0f, 0.0f, 0.0f};
        if (I4 && present && s < K) {
            /* int4: rows of octet oa (A rows 0-7) and ob (8-15), blocks 8 hd .. 8 hd + 7 */
            const uint8_t *dw = g53_dm_uptr(ex.down.w);
            const uint8_t *pl = dw + ((size_t)(m < 8 ? oa : ob) * G53_DEC_NBI + 8 * hd) * 512 + (grp * 8 + (m & 7)) * 16;
            const float *sb = ex.down.s + ((size_t)(grp < 2 ? oa : ob) * G53_DEC_NBI + 8 * hd) * 16 +
                              (m < 6 ? m / 3 : 0) * 8 + 4 * (grp & 1);
            load_all();
            __builtin_amdgcn_sched_barrier(0);
            constexpr int NB = G53_DEC_NBI / 2;
            g53_u4 r[NB];
            float4 stp[NB];
#pragma unroll
            for (int j = 0; j < NB; j++) {
                r[j] = G53_DM_LD((g53_mgv4 *)(pl + 512 * j));
                stp[j] = *(g53_mgf4 *)(sb + 16 * j);
            }
            stage_act();
            g53_m4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
            const uint8_t *bq0 = myaq + grp * 128 + g53_dm_i4_slot(m, grp) * 32;
            const uint8_t *bs0 = myasc + grp * 16 + g53_dm_i4_sc(m);
            g53_m8i bn = *(const g53_m8i *)bq0;
            int sn = bs0[0];
#pragma unroll
            for (int kb = 0; kb < NB; kb++) {
                const g53_m8i bc = bn;
                const int sc = sn;
                if (kb + 1 < NB) {
                    bn = *(const g53_m8i *)(bq0 + (kb + 1) * G53_DM_BB);
                    sn = bs0[(kb + 1) * 64];
                }
                g53_dm_i4_mma(acc, r[kb], bc, sc, stp[kb]);
                if ((kb % G53_DM_PIN) == G53_DM_PIN - 1) asm volatile("" : "+v"(acc));
            }
            v = g53_dm_i4_colsum(acc);
        } else if (present) {
            const uint8_t *dw = g53_dm_uptr(ex.down.w);
            const uint8_t *pl = dw + (size_t)(m < 8 ? oa : ob) * (G53_DEC_NBI * 1024) + (8 * hd) * 1024 +
                                (grp * 8 + (m & 7)) * 16;
            const float *sp = ex.down.s + (size_t)(oa >> 4) * ex.down.scols + 8 * hd + (lane & 7);
            const float scv = *(const g53_gf *)sp;
            load_all();
            __builtin_amdgcn_sched_barrier(0);
            g53_mgv4 *q = (g53_mgv4 *)pl;
            constexpr int NB = G53_DEC_NBI / 2;
            g53_m8i r[NB];
#pragma unroll
            for (int j = 0; j < NB; j++) r[j] = g53_dm_ld(q + 64 * j);
            stage_act();
            g53_m4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
            const int sbits = __float_as_int(scv);
            const uint8_t *bq0 = myaq + grp * 128 + min(m, 3) * 32;
            const uint8_t *bs0 = myasc + lane;
#if G53_DM_BPIPE
            g53_m8i bn = *(const g53_m8i *)bq0;
            int sn = bs0[0];
#endif
#pragma unroll
            for (int kb = 0; kb < NB; kb++) {
                const float sd = __int_as_float(__builtin_amdgcn_readlane(sbits, kb));
#if G53_DM_BPIPE
                const g53_m8i bc = bn;
                const int sc = sn;
                if (kb + 1 < NB) {
                    bn = *(const g53_m8i *)(bq0 + (kb + 1) * G53_DM_BB);
                    sn = bs0[(kb + 1) * 64];
                }
                g53_dm_mma(acc, r[kb], bc, sc, sd);
#else
                g53_dm_block(acc, r[kb], bq0 + kb * G53_DM_BB, bs0 + kb * 64, m < 3, sd);
#endif
                if ((kb % G53_DM_PIN) == G53_DM_PIN - 1) asm volatile("" : "+v"(acc));
            }
            v = g53_dm_planesum(acc);
        }
        if (t < 32) G53_MTRACE(65 + 2 * t);
        /* lanes 0, 16: rows 0-7 of octet oa; lanes 32, 48: rows 0-7 of octet ob. The halves meet
         * in LDS: the second to finish adds them, first half first */
        if (m == 0)
#pragma unroll
            for (int i = 0; i < 4; i++) dpart[dp][hd][4 * grp + i][s] = v[i];
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        G53_CBAR();
        int second = 0;
        if (lane == 0) second = g53_lds_add(&dcnt[dp][s], 1) == 1;
        if (!__builtin_amdgcn_readfirstlane(second)) continue;
        G53_CBAR();
        if (lane < 16) {
            const int oo = lane < 8 ? oa : ob;
            if (lane < 8 || ob != oa)
                cvals[(oo - do_lo) * 8 + (lane & 7)][s] = dpart[dp][0][lane][s] + dpart[dp][1][lane][s];
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        G53_CBAR();
        int fin = 0;
        if (lane == 0) fin = g53_lds_add(&ndone, 1) == n_dall - 1;
        if (__builtin_amdgcn_readfirstlane(fin)) {
            /* the combine (reference :1329-1340): double in slot order, then the shared expert */
            G53_CBAR();
            if (g53_lds_ld(&routed) == 0 && !g53_wait_lds(&routed, 1) && lane == 0) g53_flag_err(a.err, 1);
            if (lane < n_do * 8) {
                double acc = 0.0;
                for (int j = 0; j < K; j++) acc = acc + (double)sw[j] * (double)cvals[lane][j];
                float out = (float)acc;
                if (hs) out = out + cvals[lane][K];
                a.out[do_lo * 8 + lane] = out;
            }
            G53_MTRACE(3);
        }
    }
    G53_MTRACE(4 + (w & 7));
}

/* ------------------------------------------------------------------ host side ---- */
static int g_dm_grid = -1;
static unsigned g_dm_epoch = 0;
static void *g_dm_buf = nullptr;
static size_t g_dm_buf_bytes = 0;
static g53_u64 *g_dm_trace = nullptr;

extern "C" int g53h_set_mfma_decode_trace(void *dev_buf)
{
    g_dm_trace = (g53_u64 *)dev_buf;
    return 0;
}

static int dm_takes(const G53hMoeLayer *L, const int *idx_in)
{
    return (L->tiled == 2 || L->tiled == 4) && L->block_c == 128 && L->hidden == G53_DEC_E && L->inter == G53_DEC_I &&
           (idx_in || (L->router_dt == 1 && L->router)) && L->topk >= 1 && L->topk <= G53_DEC_MAXK &&
           L->n_experts >= 1 && L->n_experts <= G53_DEC_MAXNE;
}

static int dm_size_grid(void)
{
    if (g_dm_grid < 0) {
        const int cus = g53h_num_cus();
        int per = 0;
        g_dm_grid = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, (const void *)k_dec_mfma<false>, G53_DM_NT, 0) != hipSuccess)
            (void)hipGetLastError();
        else if (per >= 1 && cus >= 128 && cus <= 512)
            g_dm_grid = cus;
    }
    return g_dm_grid;
}

#define G53_DM_OFF_ACT ((size_t)G53_DEC_MAXNE * 8)
#define G53_DM_ACT_COPY ((size_t)(G53_DEC_MAXK + 1) * G53_DEC_I * 8)

/* Launch k_dec_mfma; returns 1 when the layer is not one it takes (the caller falls back). */
int g53h_decode_mtiled(float *out, const float *x, const G53hMoeLayer *L, int *idx_out, float *w_out,
                       const int *idx_in, const float *w_in)
{
    if (!dm_takes(L, idx_in) || !dm_size_grid()) return 1;
    if (!g_dm_buf) {
        const size_t bytes = G53_DM_OFF_ACT + G53_DM_ROT * G53_DM_ACT_COPY;
        G53_TRY(hipMalloc(&g_dm_buf, bytes));
        G53_TRY(hipMemset(g_dm_buf, 0, bytes));
        G53_TRY(hipDeviceSynchronize());
        g_dm_buf_bytes = bytes;
        g_dm_epoch = 0;
    }
    if (++g_dm_epoch == 0) {                             /* wrapped: clear and start over */
        G53_TRY(hipStreamSynchronize(g53h_stream()));
        G53_TRY(hipMemset(g_dm_buf, 0, g_dm_buf_bytes));
        G53_TRY(hipDeviceSynchronize());
        g_dm_epoch = 1;
    }
    char *buf = (char *)g_dm_buf;
    G53MfmaArgs e;
    e.out = out; e.x = x; e.router = (const uint16_t *)L->router; e.bias = L->bias;
    e.experts = L->experts; e.shared = L->shared;
    e.score = (g53_u64 *)buf;
    e.act = (g53_u64 *)(buf + G53_DM_OFF_ACT + (g_dm_epoch % G53_DM_ROT) * G53_DM_ACT_COPY);
    e.err = g53h_errblock() + 1; e.idx_out = idx_out; e.w_out = w_out; e.idx_in = idx_in; e.w_in = w_in;
    e.NE = L->n_experts; e.K = L->topk; e.norm_topk = L->norm_topk; e.epoch = g_dm_epoch;
    e.spin = g53h_spin_limit(); e.routed_scale = L->routed_scale; e.limit = L->swiglu_limit; e.trace = g_dm_trace;
    e.nrouter = nullptr; e.nbias = nullptr; e.nscore = e.nchoice = nullptr;
    G53NextReq *nq = g53h_next_req();
    const int rows = (L->n_experts + g_dm_grid - 1) / g_dm_grid;
    /* the next layer's scores by spare waves: a bf16 router on this x, and at least two set-up
     * waves left (router rows + next rows + the routing wave + 2 <= the workgroup's waves) */
    if (nq->armed && nq->dt == 1 && nq->x == x && nq->NE == L->n_experts && nq->E == G53_DEC_E &&
        (idx_in ? 0 : rows) + rows + 3 <= G53_DM_NW) {
        float *nb = g53h_next_buf();
        if (!nb) return -1;
        e.nrouter = (const uint16_t *)nq->gate; e.nbias = nq->bias; e.nchoice = nb; e.nscore = nb + 1024;
        nq->armed = 0;
    }
    g53h_prof_mark(G53_PROF_START);
    if (L->tiled == 4)                 /* int4 MFMA-tiled routed experts */
        hipLaunchKernelGGL(k_dec_mfma<true>, dim3(g_dm_grid), dim3(G53_DM_NT), 0, g53h_stream(), e);
    else
        hipLaunchKernelGGL(k_dec_mfma<false>, dim3(g_dm_grid), dim3(G53_DM_NT), 0, g53h_stream(), e);
    g53h_prof_mark(G53_PROF_FUSED);
    G53_LAUNCHED("k_dec_mfma");
    return 0;
}
