/* g53h_dectile.hip - single-token decode of one MoE layer in one launch, over experts stored
 * in the octet-tiled layout (k_dec_tiled; include/g53h.h, G53H_MAT_TILED).
 *
 * Reference: src/core/glm53f_ops.c:1144-1342 (moe_chunk) at T = 1, with the router of
 * :945-976, the FP8 matrix-vector product of :185-228, the SwiGLU of :486-494 and the combine
 * of :1329-1340, bit for bit.
 *
 * The work of a layer is cut into tasks, each one wave streaming one row octet's 1 KB units:
 *   G  one row octet of one slot's gate or up matrix (32 units, 32 KB): 8 row sums; the gate
 *      and up tasks of an octet meet in LDS, and the second to finish forms the SwiGLU and
 *      publishes the octet's 8 activations;
 *   D  two row octets of one slot's down matrix (16 + 16 units, 32 KB, all in flight before
 *      the task waits for the slot's activations): 16 contributions.
 * A unit load is one 64-lane load of 16 bytes per lane, 1 KB of consecutive HBM bytes, and it
 * leaves in every lane exactly the 16 codes of one of the reference's eight fp32 accumulators
 * of one row and block; the lane multiplies them in column order, the eight lanes of a row join
 * their accumulators by the reference's pairwise double tree through DPP exchanges, scale the
 * block sum in double and add it to the row's double sum in block order (a D task runs its two
 * octets' units of one block through one tree: half of a row's lanes finish each octet's block
 * sum). Nothing is traded through LDS and every load instruction of the kernel reads whole 1 KB
 * runs.
 *
 * Workgroup b of G (one per CU) owns gate/up octets [256 b / G, 256 (b+1) / G) and down octets
 * [512 b / G, 512 (b+1) / G) of every slot: its down rows' contributions of every slot stay in
 * its LDS, so the weighted combine of its output rows is local. Its tasks, taken in order by its
 * waves through an LDS counter: the shared expert's G tasks, its D tasks, the routed slots' G
 * tasks slot by slot, their D tasks. The routing (the one wait on other workgroups before the
 * routed slots can start) is taken by one wave while the others stream the shared expert, and a
 * D task issues its first code loads before it waits for its slot's activations.
 *
 * Cross-workgroup values (scores, activations) are words tagged with the launch's epoch,
 * published by atomic exchange and read coherently until current (g53h_xwg.h). Every wait is
 * bounded; one that runs out sets an error flag and the wave goes on, so the grid drains. */
#include <hip/hip_runtime.h>
#include <math.h>
#include <type_traits>

#include "g53h.h"
#include "g53h_core.h"
#include "g53h_gemv.h"
#include "g53h_kern.h"
#include "g53h_runtime.h"
#include "g53h_xwg.h"

#ifndef G53_DT_NW
#define G53_DT_NW 8                /* waves per workgroup                                */
#endif
#ifndef G53_DT_P
#define G53_DT_P 16                /* units (1 KB) in flight per wave                     */
#endif
#define G53_DT_NT (64 * G53_DT_NW)
#define G53_DT_PAD 20              /* floats per 16-value run of a vector in LDS (banks)  */
#define G53_DT_BLK (8 * G53_DT_PAD)/* floats per 128-column block of a vector in LDS      */
#ifndef G53_DT_APAD
#define G53_DT_APAD 20             /* the same for the activation vectors                */
#endif
#define G53_DT_ABLK (8 * G53_DT_APAD)
#define G53_DT_NGO (G53_DEC_I / 8) /* gate/up row octets                                 */
#define G53_DT_NDO (G53_DEC_E / 8) /* down row octets                                    */
#define G53_DT_MAXGO 2             /* per workgroup, grid >= 128                         */
#define G53_DT_MAXDO 4
#define G53_DT_DTAB 24576          /* bytes of the expert table staged in LDS            */
#define G53_DT_ROT 16              /* copies of the tagged activations, used in rotation  */

#ifndef G53_DT_NTW
#define G53_DT_NTW 1
#endif
#if G53_DT_NTW
#define G53_DT_LD(p) __builtin_nontemporal_load(p)  /* codes are read once: stream past the caches */
#else
#define G53_DT_LD(p) (*(p))
#endif
#if defined(__HIP_DEVICE_COMPILE__)
typedef __attribute__((address_space(1))) const g53_u4 g53_gv4t;
typedef __attribute__((address_space(1))) const float4 g53_gf4;
#else
typedef const g53_u4 g53_gv4t;
typedef const float4 g53_gf4;
#endif

struct G53TiledArgs {
    float *out;
    const float *x;
    const uint16_t *router;        /* bf16 [NE][E]                                       */
    const float *bias;
    const G53hExpert *experts;
    const G53hExpert *shared;
    g53_u64 *score;                /* [NE] tagged scores                                 */
    g53_u64 *act;                  /* [MAXK + 1][I] tagged activations, slot K = shared  */
    int *err;
    int *idx_out;
    float *w_out;
    const int *idx_in;             /* the routing when the caller has done it (or NULL)   */
    const float *w_in;
    int NE, K, norm_topk;
    unsigned epoch;
    float routed_scale, limit;
    int spin;                      /* polls before a wait on another workgroup gives up */
    g53_u64 *trace;                /* optional: [grid][32] timestamps                    */
    const uint16_t *nrouter;       /* optional: the next layer's bf16 router [NE][E] and bias, */
    const float *nbias;            /* whose scores (choice = score + bias) spare waves write */
    float *nscore, *nchoice;       /* to nscore / nchoice [NE] (the prediction's input)      */
};

/* A descriptor this kernel can stream: the released shapes, 128 x 128 blocks, every matrix
 * octet-tiled. */
__device__ __forceinline__ bool g53_desc_tiled(const G53hExpert &e)
{
    return g53_desc_ok(e) && (e.gate.flags & G53H_MAT_TILED) && (e.up.flags & G53H_MAT_TILED) &&
           (e.down.flags & G53H_MAT_TILED);
}

__device__ __forceinline__ int g53_sigma(int p) { return ((p & 1) << 2) | (p & 2) | (p >> 2); }

/* One lane's accumulator of one unit: its 16 codes times the 16 matching inputs, in column
 * order (reference src/core/glm53f_ops.c:197-205: a[l] = fmaf(w, x, a[l]), j += 8). */
__device__ __forceinline__ float g53_oct_acc(const g53_u4 &c, const float4 (&xv)[4])
{
    float a = 0.0f;
    const uint32_t d[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const g53_f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)d[k], false);
        const g53_f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)d[k], true);
        a = __builtin_fmaf(lo[0], xv[k].x, a);
        a = __builtin_fmaf(lo[1], xv[k].y, a);
        a = __builtin_fmaf(hi[0], xv[k].z, a);
        a = __builtin_fmaf(hi[1], xv[k].w, a);
    }
    return a;
}

template <int CTRL>
__device__ __forceinline__ double g53_dpp64(double v)
{
    const g53_u64 u = __builtin_bit_cast(g53_u64, v);
    const int lo = __builtin_amdgcn_mov_dpp((int)(uint32_t)u, CTRL, 0xf, 0xf, true);
    const int hi = __builtin_amdgcn_mov_dpp((int)(uint32_t)(u >> 32), CTRL, 0xf, 0xf, true);
    return __builtin_bit_cast(double, ((g53_u64)(uint32_t)hi << 32) | (uint32_t)lo);
}

/* The block sum of the row whose eight accumulators the lanes of this octet hold (runs p =
 * accumulators 0 4 2 6 1 5 3 7): ((a0 + a4) + (a2 + a6)) + ((a1 + a5) + (a3 + a7)) in double
 * (reference :206-209), neighbours (DPP quad_perm 1032), then pairs (quad_perm 2301), then the
 * two halves (row_half_mirror). Every lane of the octet ends with the same value. */
__device__ __forceinline__ double g53_oct_tree(float a)
{
    double t = (double)a;
    t = t + g53_dpp64<0xB1>(t);
    t = t + g53_dpp64<0x4E>(t);
    t = t + g53_dpp64<0x141>(t);
    return t;
}

struct G53NoWait {
    __device__ void operator()() const {}
};

__device__ __forceinline__ const uint8_t *g53_uniform_ptr(const uint8_t *p)
{
    const g53_u64 v = (g53_u64)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const uint8_t *)(uintptr_t)(((g53_u64)hi << 32) | lo);
}

/* Stream one row octet's NU consecutive units (pu: its first unit; this lane's 16 bytes at
 * + 16 lane), unit u against block u of the vector at xv (this lane's run of it in LDS), and
 * return the octet rows' sums in block order (the same in every lane of a row's octet). sp
 * points lane u at unit u's block scale. P units are in flight; two are multiplied at a time
 * (independent block sums), their scaled sums then added in order. ready() runs after the
 * first loads are issued and before the first multiply (the vector may still be on its way into
 * LDS). */
template <int NU, int VBLK, class Ready>
__device__ __forceinline__ double g53_oct_stream(const uint8_t *pu, const float *sp, const float *xv, int lane,
                                                 const Ready &ready)
{
    constexpr int P = G53_DT_P < NU ? G53_DT_P : NU;
    static_assert(P % 2 == 0 && NU % P == 0, "units in flight");
    /* the block scales are loaded before the codes, so that waiting for them never waits for
     * codes still in flight */
    const float scv = *(const g53_gf *)sp;
    __builtin_amdgcn_sched_barrier(0);
    g53_gv4t *q = (g53_gv4t *)(g53_uniform_ptr(pu) + 16 * lane);
    g53_u4 r[P];
#pragma unroll
    for (int j = 0; j < P; j++) r[j] = G53_DT_LD(q + 64 * j);
    ready();
    double acc = 0.0;
    const int sbits = __float_as_int(scv);
    auto pair = [&](int u, int j, bool refill) {
        const float4 *x0 = (const float4 *)(xv + u * VBLK), *x1 = (const float4 *)(xv + (u + 1) * VBLK);
        const float4 xa[4] = {x0[0], x0[1], x0[2], x0[3]};
        const float4 xb[4] = {x1[0], x1[1], x1[2], x1[3]};
        const float fa = g53_oct_acc(r[j], xa), fb = g53_oct_acc(r[j + 1], xb);
        if (refill) {
            r[j] = G53_DT_LD(q + 64 * (u + P));
            r[j + 1] = G53_DT_LD(q + 64 * (u + 1 + P));
        }
        const double ta = g53_oct_tree(fa), tb = g53_oct_tree(fb);
        acc = acc + ta * (double)__int_as_float(__builtin_amdgcn_readlane(sbits, u));
        acc = acc + tb * (double)__int_as_float(__builtin_amdgcn_readlane(sbits, u + 1));
    };
    /* steady state: multiply two units, refill their registers P units ahead */
#pragma unroll 1
    for (int u0 = 0; u0 < NU - P; u0 += P) {
#pragma unroll
        for (int j = 0; j < P; j += 2) pair(u0 + j, j, true);
    }
#pragma unroll
    for (int j = 0; j < P; j += 2) pair(NU - P + j, j, false);
    return acc;
}

/* Two units' block sums through one tree: each lane holds accumulator sigma(p) of unit A (fa)
 * and of unit B (fb). Lanes of role 0 (run p with (p ^ p >> 2) & 1 == 0) end with A's block
 * sum, lanes of role 1 with B's. The first level trades one float with the neighbour (which
 * has the other role) and adds in the lane; the pairs and the halves (quad_perm 2301,
 * row_half_mirror) join lanes of the same role. The additions and their grouping are those
 * of g53_oct_tree, ((a0 + a4) + (a2 + a6)) + ((a1 + a5) + (a3 + a7)) (reference :206-209). */
__device__ __forceinline__ double g53_oct_tree2(float fa, float fb, bool r1)
{
    const float send = r1 ? fa : fb, own = r1 ? fb : fa;
    const float got = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(send), 0xB1, 0xf, 0xf, true));
    double t = (double)own + (double)got;
    t = t + g53_dpp64<0x4E>(t);
    t = t + g53_dpp64<0x141>(t);
    return t;
}

/* The same for two row octets at once (pa, pb), unit u of both against block u: their sums in
 * block order come back in acc_a and acc_b. sp points lane u at sequence a's unit u scale and
 * lane 32 + u at b's. All 2 NU units are in flight before ready() runs. */
template <int NU, int VBLK, class Ready>
__device__ __forceinline__ void g53_oct_stream2(const uint8_t *pa, const uint8_t *pb, const float *sp, const float *xv,
                                                int lane, const Ready &ready, double &acc_a, double &acc_b)
{
    const float scv = *(const g53_gf *)sp;
    __builtin_amdgcn_sched_barrier(0);
    g53_gv4t *qa = (g53_gv4t *)(g53_uniform_ptr(pa) + 16 * lane);
    g53_gv4t *qb = (g53_gv4t *)(g53_uniform_ptr(pb) + 16 * lane);
    g53_u4 ra[NU], rb[NU];
#pragma unroll
    for (int u = 0; u < NU; u++) {
        ra[u] = G53_DT_LD(qa + 64 * u);
        rb[u] = G53_DT_LD(qb + 64 * u);
    }
    ready();
    const int sbits = __float_as_int(scv);
    /* one tree for both units; this lane's role keeps one octet's sum */
    const int pr = lane & 7;
    const bool r1 = ((pr ^ (pr >> 2)) & 1) != 0;
    double acc = 0.0;
#pragma unroll
    for (int u = 0; u < NU; u++) {
        const float4 *xr = (const float4 *)(xv + u * VBLK);
        const float4 x4[4] = {xr[0], xr[1], xr[2], xr[3]};
        const float fa = g53_oct_acc(ra[u], x4), fb = g53_oct_acc(rb[u], x4);
        const double t = g53_oct_tree2(fa, fb, r1);
        const float sa = __int_as_float(__builtin_amdgcn_readlane(sbits, u));
        const float sb = __int_as_float(__builtin_amdgcn_readlane(sbits, 32 + u));
        acc = acc + t * (double)(r1 ? sb : sa);
    }
    const double other = g53_dpp64<0xB1>(acc);          /* the neighbour has the other role */
    acc_a = r1 ? other : acc;
    acc_b = r1 ? acc : other;
}

/* ----------------------------------------------------------- int4 experts ---- */
/* A descriptor of int4 codes in the int4-tiled layout (include/g53h.h, G53H_MAT_I4T) with the
 * released shapes and one step per row and 64 columns. */
__device__ __forceinline__ bool g53_desc_i4t(const G53hExpert &e)
{
    const G53hMat *m[3] = {&e.gate, &e.up, &e.down};
    const int rows[3] = {G53_DEC_I, G53_DEC_I, G53_DEC_E}, cols[3] = {G53_DEC_E, G53_DEC_E, G53_DEC_I};
    bool ok = true;
    for (int i = 0; i < 3; i++)
        ok = ok && m[i]->w && m[i]->s && (m[i]->flags & G53H_MAT_I4) && (m[i]->flags & G53H_MAT_I4T) &&
             m[i]->rows == rows[i] && m[i]->cols == cols[i] && m[i]->bc == 64 && m[i]->scols == cols[i] / 64;
    return ok;
}

/* One lane's accumulator of one 64-column group: its 8 levels (nibbles of d, the low one first)
 * times the 8 matching inputs in column order, a = fmaf((float)(level - 8), x, a) (reference
 * src/core/glm53f_ops.c:270-276). level - 8 is the 4-bit two's complement of level ^ 8. */
__device__ __forceinline__ float g53_i4_acc(uint32_t d, const float4 &x0, const float4 &x1)
{
    const uint32_t s = d ^ 0x88888888u;
    const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) a = __builtin_fmaf((float)((int)(s << (28 - 4 * i)) >> 28), xv[i], a);
    return a;
}

/* The inputs of group g (0..3) of 256-column unit u for this lane: block 2 u + g / 2 of the
 * vector tiled in LDS (run of 16 at xv, VBLK floats per block), half g % 2 of the run. */
template <int VBLK>
__device__ __forceinline__ void g53_i4_x(const float *xv, int u, int g, float4 &x0, float4 &x1)
{
    const float4 *r = (const float4 *)(xv + (2 * u + (g >> 1)) * VBLK + 8 * (g & 1));
    x0 = r[0];
    x1 = r[1];
}

#ifndef G53_DT_P4
#define G53_DT_P4 8                /* int4 G tasks: units in flight per wave               */
#endif

/* Stream one int4 row octet's NU units (pu: its first unit; this lane's 16 bytes at + 16 lane),
 * unit u's four groups against blocks 2 u, 2 u + 1 of the vector; the row's double sum over its
 * groups in order (reference :246-292), the same in every lane of the row's octet. srow: this
 * lane's row of steps (float4 u = unit u's four). */
template <int NU, int VBLK, class Ready>
__device__ __forceinline__ double g53_i4_stream(const uint8_t *pu, const float *srow, const float *xv, int lane,
                                                const Ready &ready)
{
    constexpr int P = G53_DT_P4 < NU ? G53_DT_P4 : NU;
    static_assert(NU % P == 0, "units in flight");
    g53_gv4t *q = (g53_gv4t *)(g53_uniform_ptr(pu) + 16 * lane);
    const float4 *sq = (const float4 *)srow;
    g53_u4 r[P];
    float4 st[P];
#pragma unroll
    for (int j = 0; j < P; j++) { r[j] = G53_DT_LD(q + 64 * j); st[j] = *(const g53_gf4 *)(sq + j); }
    ready();
    const int pr = lane & 7;
    const bool r1 = ((pr ^ (pr >> 2)) & 1) != 0;
    double acc = 0.0;
    auto unit = [&](int u, int j, bool refill) {
        const uint32_t d[4] = {r[j].x, r[j].y, r[j].z, r[j].w};
        const float sv[4] = {st[j].x, st[j].y, st[j].z, st[j].w};
        float f[4];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            float4 x0, x1;
            g53_i4_x<VBLK>(xv, u, g, x0, x1);
            f[g] = g53_i4_acc(d[g], x0, x1);
        }
        if (refill) {
            r[j] = G53_DT_LD(q + 64 * (u + P));
            st[j] = *(const g53_gf4 *)(sq + u + P);
        }
        /* groups (0, 1) and (2, 3) through one tree each; then each lane takes the other role's
         * sum from its neighbour, and the row adds the four in order */
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const double t = g53_oct_tree2(f[2 * h], f[2 * h + 1], r1);
            const double o = g53_dpp64<0xB1>(t);
            const double ta = r1 ? o : t, tb = r1 ? t : o;
            acc = acc + ta * (double)sv[2 * h];
            acc = acc + tb * (double)sv[2 * h + 1];
        }
        /* one unit at a time: the compiler would otherwise hoist every unit's input reads */
        asm volatile("" : "+v"(acc));
    };
#pragma unroll 1
    for (int u0 = 0; u0 < NU - P; u0 += P) {
#pragma unroll
        for (int j = 0; j < P; j++) unit(u0 + j, j, true);
    }
#pragma unroll
    for (int j = 0; j < P; j++) unit(NU - P + j, j, false);
    return acc;
}

/* Two int4 row octets at once (pa, pb): group g of unit u of both through one tree; lanes of role
 * 0 keep octet a's sums, role 1 octet b's (srow: this lane's row of steps in its role's octet).
 * All 2 NU units are in flight before ready() runs. */
template <int NU, int VBLK, class Ready>
__device__ __forceinline__ void g53_i4_stream2(const uint8_t *pa, const uint8_t *pb, const float *srow, const float *xv,
                                               int lane, const Ready &ready, double &acc_a, double &acc_b)
{
    g53_gv4t *qa = (g53_gv4t *)(g53_uniform_ptr(pa) + 16 * lane);
    g53_gv4t *qb = (g53_gv4t *)(g53_uniform_ptr(pb) + 16 * lane);
    const float4 *sq = (const float4 *)srow;
    constexpr int SR = 3;                                /* units of steps in flight */
    g53_u4 ra[NU], rb[NU];
    float4 st[SR];
#pragma unroll
    for (int u = 0; u < NU; u++) {
        ra[u] = G53_DT_LD(qa + 64 * u);
        rb[u] = G53_DT_LD(qb + 64 * u);
    }
#pragma unroll
    for (int u = 0; u < SR - 1; u++) st[u] = *(const g53_gf4 *)(sq + u);
    ready();
    const int pr = lane & 7;
    const bool r1 = ((pr ^ (pr >> 2)) & 1) != 0;
    double acc = 0.0;
#pragma unroll
    for (int u = 0; u < NU; u++) {
        if (u + SR - 1 < NU) st[(u + SR - 1) % SR] = *(const g53_gf4 *)(sq + u + SR - 1);
        const uint32_t da[4] = {ra[u].x, ra[u].y, ra[u].z, ra[u].w};
        const uint32_t db[4] = {rb[u].x, rb[u].y, rb[u].z, rb[u].w};
        const float sv[4] = {st[u % SR].x, st[u % SR].y, st[u % SR].z, st[u % SR].w};
#pragma unroll
        for (int g = 0; g < 4; g++) {
            float4 x0, x1;
            g53_i4_x<VBLK>(xv, u, g, x0, x1);
            const float fa = g53_i4_acc(da[g], x0, x1), fb = g53_i4_acc(db[g], x0, x1);
            const double t = g53_oct_tree2(fa, fb, r1);
            acc = acc + t * (double)sv[g];
        }
        asm volatile("" : "+v"(acc));            /* one unit at a time (see g53_i4_stream) */
    }
    const double other = g53_dpp64<0xB1>(acc);          /* the neighbour has the other role */
    acc_a = r1 ? other : acc;
    acc_b = r1 ? acc : other;
}

#define G53_TTRACE(k) do { if (a.trace && lane == 0) \
    a.trace[(size_t)blockIdx.x * 192 + (k)] = __builtin_amdgcn_s_memrealtime(); } while (0)

/* I4: the routed experts are int4, int4-tiled (G53H_MAT_I4T; the reference's --experts int4),
 * streamed by g53_i4_stream / g53_i4_stream2; the shared expert stays FP8 octet-tiled. */
template <bool I4>
__global__ void __launch_bounds__(G53_DT_NT, 1) k_dec_tiled(G53TiledArgs a)
{
    __shared__ __attribute__((aligned(16))) float xs[G53_DEC_NBE * G53_DT_BLK];          /* x, tiled  */
    __shared__ __attribute__((aligned(16))) float actw[G53_DT_NW][G53_DEC_NBI * G53_DT_ABLK];
    __shared__ __attribute__((aligned(16))) uint2 dtab[G53_DT_DTAB / 8];
    __shared__ G53hExpert st[G53_DEC_MAXK + 1];
    __shared__ float biasl[G53_DEC_MAXNE];
    __shared__ float cvals[G53_DT_MAXDO * 8][G53_DEC_MAXK + 1];
    __shared__ float guv[G53_DEC_MAXK + 1][G53_DT_MAXGO][2][8];   /* gate / up row sums     */
    __shared__ int gucnt[G53_DEC_MAXK + 1][G53_DT_MAXGO];
    __shared__ float sw[64];
    __shared__ int sidx[16], ebuf[64];
    __shared__ uint32_t kbuf[64];
    __shared__ uint64_t etab[32];
    __shared__ int qctr, ndone, routed, nrouted, inited;

    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int o = lane >> 3, p = lane & 7;
    const int K = a.K, hs = a.shared ? 1 : 0;
    const int G = gridDim.x, b = blockIdx.x;
    const int go_lo = G53_DT_NGO * b / G, n_go = G53_DT_NGO * (b + 1) / G - go_lo;
    const int do_lo = G53_DT_NDO * b / G, n_do = G53_DT_NDO * (b + 1) / G - do_lo;
    /* tasks: per slot its G tasks (gate and up of each owned octet) and its D tasks (pairs of
     * owned down octets); a D task has all its codes in flight before it waits for its slot's
     * activations */
    const int ng = 2 * n_go, nd = (n_do + 1) >> 1, nslot = hs + K;
    int n_task = 0;
    const int nR = a.idx_in ? 0 : (a.NE > b ? (a.NE - 1 - b) / G + 1 : 0);
    const int nN = a.nrouter ? (a.NE > b ? (a.NE - 1 - b) / G + 1 : 0) : 0;   /* next-layer rows */
    const int words = (int)(sizeof(G53hExpert) / 4);
#ifdef G53_DT_NOSTAGE
    const bool dstage = false;
#else
    const bool dstage = a.NE * (int)sizeof(G53hExpert) <= G53_DT_DTAB;
#endif
    const int n_setup = G53_DT_NW - 1 - nR - nN;   /* waves that set up the workgroup's LDS */

    G53_TTRACE(0);
    if (threadIdx.x == 0) { qctr = 0; ndone = 0; routed = 0; nrouted = 0; inited = 0; }
    __syncthreads();
    /* router rows first: waves 0 .. nR-1 take rows b, b + G, ... */
    g53_u4 cr[8];
    /* the waves on the routing's critical path (router rows, the routing wave) issue ahead of
     * the streaming waves that share their SIMD */
    if (w < nR || w == G53_DT_NW - 1) __builtin_amdgcn_s_setprio(3);
    if (w < nR) {
        g53_gv4t *q = (g53_gv4t *)(a.router + (size_t)(b + w * G) * G53_DEC_E + lane * 64);
#pragma unroll
        for (int k = 0; k < 8; k++) cr[k] = q[k];
        /* the score of expert b + w G, published at once (x read straight from memory), so
         * that the routing does not wait for the workgroup's set-up */
        const double d = g53_router_row(cr, a.x, lane);
        if (lane == 0) g53_st_tag(a.score + b + w * G, g53_tag(a.epoch, g53_sigmoidf_tab((float)d, g53_exp2_tab_dev)));
        if (w == 0) G53_TTRACE(2);
        __builtin_amdgcn_s_setprio(0);
    } else if (w < nR + nN) {
        /* the next layer's router row b + (w - nR) G on the same x: its score and choice for the
         * prediction (the arithmetic of k_router_scores, bit for bit) */
        const int e = b + (w - nR) * G;
        g53_gv4t *q = (g53_gv4t *)(a.nrouter + (size_t)e * G53_DEC_E + lane * 64);
#pragma unroll
        for (int k = 0; k < 8; k++) cr[k] = q[k];
        const double d = g53_router_row(cr, a.x, lane);
        if (lane == 0) {
            const float sc = g53_sigmoidf_tab((float)d, g53_exp2_tab_dev);
            a.nscore[e] = sc;
            a.nchoice[e] = sc + a.nbias[e];
        }
    } else if (w < G53_DT_NW - 1) {
        /* the set-up, by the waves between the router rows and the routing wave: every load
         * is issued before the first store into LDS; all waves start once it is done */
        const int ti = threadIdx.x - 64 * (nR + nN), nt = (G53_DT_NW - 1 - nR - nN) * 64;
        constexpr int XPER = 8;                             /* nt >= 128 */
        float4 xv[XPER];
        /* the expert table too, so that the routing picks the chosen descriptors from LDS */
        constexpr int DPER = 8;
        const int n8 = dstage ? a.NE * (int)(sizeof(G53hExpert) / 8) : 0;
        const uint2 *t8 = (const uint2 *)a.experts;
        uint2 dv[DPER];
#pragma unroll
        for (int k = 0; k < DPER; k++) dv[k] = ti + k * nt < n8 ? t8[ti + k * nt] : make_uint2(0u, 0u);
        int dw = 0;
        if (ti < words && hs) dw = ((const int *)a.shared)[ti];
        const uint64_t et = ti < 32 ? g53_exp2_tab_dev[ti] : 0;
#pragma unroll
        for (int k = 0; k < XPER; k++)
            xv[k] = ti + k * nt < G53_DEC_E / 4 ? ((const float4 *)a.x)[ti + k * nt] : make_float4(0.f, 0.f, 0.f, 0.f);
        if (ti < words) ((int *)&st[K])[ti] = dw;
#pragma unroll
        for (int k = 0; k < DPER; k++)
            if (ti + k * nt < n8) dtab[ti + k * nt] = dv[k];
        for (int q = ti + DPER * nt; q < n8; q += nt) dtab[q] = t8[q];        /* few set-up waves */
        if (ti < (G53_DEC_MAXK + 1) * G53_DT_MAXGO) (&gucnt[0][0])[ti] = 0;
        if (ti < 32) etab[ti] = et;
        /* x into LDS, tiled like the codes: run p of block bb holds x[bb*128 + sigma(p) + 8i] */
#pragma unroll
        for (int k = 0; k < XPER; k++) {
            if (ti + k * nt >= G53_DEC_E / 4) break;
            const float vv[4] = {xv[k].x, xv[k].y, xv[k].z, xv[k].w};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int c = 4 * (ti + k * nt) + q, bb = c >> 7, cc = c & 127;
                xs[bb * G53_DT_BLK + g53_sigma(cc & 7) * G53_DT_PAD + (cc >> 3)] = vv[q];
            }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        G53_CBAR();
        if (lane == 0) g53_lds_add(&inited, 1);
        if (w == G53_DT_NW - 2) G53_TTRACE(15);
        G53_TTRACE(128 + w);
    }
    if (w != G53_DT_NW - 1 && !g53_wait_lds(&inited, n_setup) && lane == 0) g53_flag_err(a.err, 1);
    G53_TTRACE(144 + w);

    /* the routing: top-k, weights, the chosen descriptors (reference :945-976) */
    if (w == G53_DT_NW - 1) {

        g53_u64 t_seen = 0, t_tau = 0, t_rank = 0;
        int n_polls = 0;
        bool ok = true;
        if (a.idx_in) {                               /* routed by the caller */
            if (lane < K) { sidx[lane] = a.idx_in[lane]; sw[lane] = a.w_in[lane]; }
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();
        } else if (a.NE <= 64 * 5)
            ok = g53_route_wave<5>(a.score, biasl, a.NE, K, a.norm_topk, a.routed_scale, a.epoch, sidx, sw, kbuf, ebuf,
                                   a.err, lane, t_seen, n_polls, t_tau, t_rank, a.spin, &nrouted, nullptr, a.bias);
        else
            ok = g53_route_wave<G53_DEC_MAXNE / 64>(a.score, biasl, a.NE, K, a.norm_topk, a.routed_scale, a.epoch,
                                                    sidx, sw, kbuf, ebuf, a.err, lane, t_seen, n_polls, t_tau, t_rank, a.spin, &nrouted, nullptr, a.bias);
        if (!ok) {                                    /* scores missing: no routed slots */
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
        /* the routing is handed over as the chosen experts' indices; every task looks its
         * descriptor up itself */
        G53_CBAR();
        if (lane == 0) g53_lds_add(&routed, 1);
        __builtin_amdgcn_s_setprio(0);
        if (b == 0 && lane < K && !a.idx_in) {
            if (a.idx_out) a.idx_out[lane] = sidx[lane];
            if (a.w_out) a.w_out[lane] = sw[lane];
        }
        G53_TTRACE(1);
        if (a.trace && lane == 0) {
            a.trace[(size_t)blockIdx.x * 192 + 12] = t_seen;
            a.trace[(size_t)blockIdx.x * 192 + 13] = t_tau;
            a.trace[(size_t)blockIdx.x * 192 + 14] = t_rank;
        }
    }

    if (w == G53_DT_NW - 1 && !g53_wait_lds(&inited, n_setup) && lane == 0) g53_flag_err(a.err, 1);
    /* the shared expert, if unusable, is flagged and contributes zero */
    const bool shared_ok = hs && st[K].gate.w && g53_desc_tiled(st[K]);
    if (hs && st[K].gate.w && !shared_ok && b == 0 && threadIdx.x == 0) g53_flag_err(a.err, 8);
    n_task = nslot * (ng + nd);
    const int n_dall = nslot * nd;
    float *myact = actw[w];
    g53_u64 tg = 0, twait = 0, td = 0;
    /* one task (t: its number in the order); RT: a routed slot of the int4 kernel (int4 code
     * paths), else the FP8 paths. The int4 kernel runs the shared expert's tasks, then the
     * routed ones, in two loops, so that the two kinds of down task never share registers */
    auto task = [&](int t, auto rt_tag) {
        constexpr bool RT = decltype(rt_tag)::value;
        if (t < 32) G53_TTRACE(64 + 2 * t);
        /* the order: the shared expert's G tasks, its D tasks (its activations are complete
         * while the routing is still being decided), the routed slots' G tasks slot by slot,
         * their D tasks */
        int s, idx;
        bool is_g;
        const int i_sd = hs * ng, i_rg = i_sd + hs * nd, i_rd = i_rg + K * ng;
        if (t < i_sd) { s = K; is_g = true; idx = t; }
        else if (t < i_rg) { s = K; is_g = false; idx = t - i_sd; }
        else if (t < i_rd) { s = (t - i_rg) / ng; is_g = true; idx = (t - i_rg) - s * ng; }
        else { s = (t - i_rd) / nd; is_g = false; idx = (t - i_rd) - s * nd; }
        if (s < K && g53_lds_ld(&nrouted) <= s) {          /* slot s is chosen: its index is in */
            if (!g53_wait_lds(&nrouted, s + 1) && lane == 0) g53_flag_err(a.err, 1);
        }
        /* the slot's descriptor: the shared expert's in LDS; a routed one from the staged
         * table (or memory) by the chosen index; an unusable one is flagged and skipped */
        G53hExpert ex;
        bool usable;
        if (s == K) {
            ex = st[K];
            usable = shared_ok;
        } else {
            const int e = sidx[s];
            if (e >= 0 && e < a.NE) ex = dstage ? ((const G53hExpert *)dtab)[e] : a.experts[e];
            else ex.gate.w = nullptr;
            usable = ex.gate.w != nullptr && (RT ? g53_desc_i4t(ex) : g53_desc_tiled(ex));
            if (ex.gate.w && !usable && lane == 0) g53_flag_err(a.err, 8);
        }
        const bool present = __builtin_amdgcn_readfirstlane((int)usable) != 0;
        if (is_g) {
            if (!present) return;                     /* its activations are never read */
            const int ogl = idx >> 1, og = go_lo + ogl, m = idx & 1;
            const G53hMat &mat = m ? ex.up : ex.gate;
            const g53_u64 t0 = a.trace ? __builtin_amdgcn_s_memrealtime() : 0;
            double acc;
            if constexpr (RT) {
                const uint8_t *pu = mat.w + (size_t)og * (G53_DEC_E / 256 * 1024);
                const float *srow = mat.s + (size_t)(og * 8 + o) * mat.scols;
                acc = g53_i4_stream<G53_DEC_E / 256, G53_DT_BLK>(pu, srow, xs + p * G53_DT_PAD, lane, G53NoWait());
            } else {
                const uint8_t *pu = mat.w + (size_t)og * (G53_DEC_NBE * 1024);
                const float *sp = mat.s + (size_t)(og >> 4) * mat.scols + (lane & 31);
                acc = g53_oct_stream<G53_DEC_NBE, G53_DT_BLK>(pu, sp, xs + p * G53_DT_PAD, lane, G53NoWait());
            }
            if (a.trace) tg += __builtin_amdgcn_s_memrealtime() - t0;
            /* gate and up of an octet meet in LDS; the second of the two computes the SwiGLU
             * and publishes the octet's activations */
            if (p == 0) guv[s][ogl][m][o] = (float)acc;
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();
            G53_CBAR();
            int second = 0;
            if (lane == 0) second = g53_lds_add(&gucnt[s][ogl], 1) == 1;
            if (__builtin_amdgcn_readfirstlane(second)) {
                G53_CBAR();
                if (p == 0) {
                    const float v = g53_swiglu1_tab(guv[s][ogl][0][o], guv[s][ogl][1][o], a.limit, etab);
                    g53_st_tag(a.act + (size_t)s * G53_DEC_I + og * 8 + o, g53_tag(a.epoch, v));
                }
            }
            if (t < 32) G53_TTRACE(65 + 2 * t);
            return;
        }
        const int oa = do_lo + 2 * idx, ob = oa + 1 < do_lo + n_do ? oa + 1 : oa;
        float va = 0.0f, vb = 0.0f;
        if (present) {
            const uint8_t *pa = ex.down.w + (size_t)oa * (G53_DEC_NBI * 1024);
            const uint8_t *pb = ex.down.w + (size_t)ob * (G53_DEC_NBI * 1024);
            const float *sp = ex.down.s + (size_t)((lane < 32 ? oa : ob) >> 4) * ex.down.scols + (lane & 15);
            const g53_u64 t0 = a.trace ? __builtin_amdgcn_s_memrealtime() : 0;
            g53_u64 t1 = t0;
            /* the slot's activations into this wave's LDS, tiled like x, once its codes are on
             * their way: 32 consecutive values per lane, re-read until every tag is current */
            auto ready = [&]() {
                /* first the last value of every row octet (256 words, 2 KB per poll instead of
                 * the vector's 16 KB), with a growing back-off: a wait does not flood the memory
                 * system while the values are still being computed */
                const __amdgpu_buffer_rsrc_t rsl = g53_rsrc(a.act + (size_t)s * G53_DEC_I);
                int spins = 0, nap = 1;
                for (;;) {
                    g53_u64 tv[G53_DT_NGO / 64];
#pragma unroll
                    for (int k = 0; k < G53_DT_NGO / 64; k++) tv[k] = g53_ld_coh64(rsl, 8 * ((lane + 64 * k) * 8 + 7));
                    int stale = 0;
#pragma unroll
                    for (int k = 0; k < G53_DT_NGO / 64; k++) stale |= (unsigned)(tv[k] >> 32) != a.epoch;
                    if (!__ballot(stale)) break;
                    if (++spins > a.spin / 16 + 1) { if (lane == 0) g53_flag_err(a.err, 1); break; }
                    for (int q = 0; q < nap; q++) __builtin_amdgcn_s_sleep(8);
                    if (nap < 8) nap *= 2;
                }
                /* then the values through this XCD's L2 (one memory read serves its 32 CUs); a
                 * value older than this launch (a line the L2 took before it was written) is
                 * re-read coherently and stored back, which refreshes the line for the CUs of
                 * this XCD that read it later */
                g53_u64 *act_s = a.act + (size_t)s * G53_DEC_I;
                const __amdgpu_buffer_rsrc_t rs = g53_rsrc(act_s);
                const int v0 = 32 * lane, bb = v0 >> 7, c0 = v0 & 127;
                float *dst = myact + bb * G53_DT_ABLK;
                g53_gv4t *src = (g53_gv4t *)(act_s + v0);
                uint32_t pend = 0;
#pragma unroll
                for (int h = 0; h < 32; h += 8) {
                    g53_u64 tw[8];
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const g53_u4 qv = src[(h >> 1) + k];
                        tw[2 * k] = ((g53_u64)qv.y << 32) | qv.x;
                        tw[2 * k + 1] = ((g53_u64)qv.w << 32) | qv.z;
                    }
#pragma unroll
                    for (int mm = 0; mm < 8; mm++) {
                        const int cc = c0 + h + mm;
                        dst[g53_sigma(cc & 7) * G53_DT_APAD + (cc >> 3)] = __uint_as_float((uint32_t)tw[mm]);
                        if ((unsigned)(tw[mm] >> 32) != a.epoch) pend |= 1u << (h + mm);
                    }
                }
                spins = 0;
                while (__ballot(pend != 0)) {
                    if (++spins > a.spin) { if (lane == 0) g53_flag_err(a.err, 1); break; }
                    g53_backoff();
#pragma unroll
                    for (int mm = 0; mm < 32; mm++) {
                        if (!(pend & (1u << mm))) continue;
                        const g53_u64 tv = g53_ld_coh64(rs, 8 * (v0 + mm));
                        if ((unsigned)(tv >> 32) == a.epoch) {
                            const int cc = c0 + mm;
                            dst[g53_sigma(cc & 7) * G53_DT_APAD + (cc >> 3)] = __uint_as_float((uint32_t)tv);
                            act_s[v0 + mm] = tv;
                            pend &= ~(1u << mm);
                        }
                    }
                }
                __builtin_amdgcn_s_waitcnt(0xc07f);
                __builtin_amdgcn_wave_barrier();
                if (a.trace) t1 = __builtin_amdgcn_s_memrealtime();
            };
            double da, db;
            if constexpr (RT) {
                const uint8_t *qa = ex.down.w + (size_t)oa * (G53_DEC_I / 256 * 1024);
                const uint8_t *qb = ex.down.w + (size_t)ob * (G53_DEC_I / 256 * 1024);
                const bool r1 = ((p ^ (p >> 2)) & 1) != 0;      /* this lane's octet in the shared trees */
                const float *srow = ex.down.s + (size_t)((r1 ? ob : oa) * 8 + o) * ex.down.scols;
                g53_i4_stream2<G53_DEC_I / 256, G53_DT_ABLK>(qa, qb, srow, myact + p * G53_DT_APAD, lane, ready, da, db);
            } else {
                g53_oct_stream2<G53_DEC_NBI, G53_DT_ABLK>(pa, pb, sp, myact + p * G53_DT_APAD, lane, ready, da, db);
            }
            va = (float)da;
            vb = (float)db;
            if (a.trace) {
                const g53_u64 t2 = __builtin_amdgcn_s_memrealtime();
                twait += t1 - t0;
                td += t2 - t1;
            }
        }
        if (t < 32) G53_TTRACE(65 + 2 * t);
        if (p == 0) {
            cvals[(oa - do_lo) * 8 + o][s] = va;
            if (ob != oa) cvals[(ob - do_lo) * 8 + o][s] = vb;
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        G53_CBAR();
        int fin = 0;
        if (lane == 0) fin = g53_lds_add(&ndone, 1) == n_dall - 1;
        if (__builtin_amdgcn_readfirstlane(fin)) {
            /* every contribution of the workgroup's rows is in: the combine (reference
             * :1329-1340), double in slot order, then the shared expert in float */
            G53_CBAR();
            if (g53_lds_ld(&routed) == 0 && !g53_wait_lds(&routed, 1) && lane == 0) g53_flag_err(a.err, 1);
            if (lane < n_do * 8) {
                double acc = 0.0;
                for (int j = 0; j < K; j++) acc = acc + (double)sw[j] * (double)cvals[lane][j];
                float out = (float)acc;
                if (hs) out = out + cvals[lane][K];
                a.out[do_lo * 8 + lane] = out;
            }
            G53_TTRACE(3);
        }
    };
    auto claim = [&]() {
        int t = 0;
        if (lane == 0) t = g53_lds_add(&qctr, 1);
        return __builtin_amdgcn_readfirstlane(t);
    };
    {
        const int i_rg = hs * (ng + nd);                /* the first routed task */
        int t = claim();
        for (; t < n_task && (!I4 || t < i_rg); t = claim()) task(t, std::integral_constant<bool, false>());
        if constexpr (I4)
            for (; t < n_task; t = claim()) task(t, std::integral_constant<bool, true>());
    }
    G53_TTRACE(4 + (w & 7));
    if (a.trace && lane == 0 && w < 16) {
        a.trace[(size_t)blockIdx.x * 192 + 16 + w] = tg;
        a.trace[(size_t)blockIdx.x * 192 + 32 + w] = twait;
        a.trace[(size_t)blockIdx.x * 192 + 48 + w] = td;
    }
}

/* ------------------------------------------------------------------ host side ---- */
static int g_dt_grid = -1;
static unsigned g_dt_epoch = 0;
static void *g_dt_buf = nullptr;        /* tagged scores | tagged activations              */
static size_t g_dt_buf_bytes = 0;
static g53_u64 *g_dt_trace = nullptr;

extern "C" int g53h_set_tiled_decode_trace(void *dev_buf)
{
    g_dt_trace = (g53_u64 *)dev_buf;
    return 0;
}

int g53h_decode_tiled_grid(void) { return g_dt_grid; }

static int dt_takes(const G53hMoeLayer *L, const int *idx_in)
{
    return (L->tiled == 1 || L->tiled == 3) && L->block_c == 128 && L->hidden == G53_DEC_E && L->inter == G53_DEC_I &&
           (idx_in || (L->router_dt == 1 && L->router)) && L->topk >= 1 && L->topk <= G53_DEC_MAXK &&
           L->n_experts >= 1 && L->n_experts <= G53_DEC_MAXNE;
}

static int dt_size_grid(void)
{
    if (g_dt_grid < 0) {
        const int cus = g53h_num_cus();
        int per = 0;
        g_dt_grid = 0;
        int per4 = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, (const void *)k_dec_tiled<false>, G53_DT_NT, 0) !=
                hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per4, (const void *)k_dec_tiled<true>, G53_DT_NT, 0) !=
                hipSuccess) {
            (void)hipGetLastError();
        } else if (per >= 1 && per4 >= 1 && cus >= 128 && cus <= 512) {
            g_dt_grid = cus;
        }
    }
    return g_dt_grid;
}

/* Scratch of one launch: tagged scores [G53_DEC_MAXNE], then G53_DT_ROT copies of the tagged
 * activations [(G53_DEC_MAXK + 1) * G53_DEC_I], one per epoch in rotation. Tags are the epoch,
 * so the memory needs clearing only when a fresh buffer starts and when the epoch wraps. */
#define G53_DT_OFF_ACT ((size_t)G53_DEC_MAXNE * 8)
#define G53_DT_ACT_COPY ((size_t)(G53_DEC_MAXK + 1) * G53_DEC_I * 8)
#define G53_DT_SCRATCH (G53_DT_OFF_ACT + G53_DT_ROT * G53_DT_ACT_COPY)

static void dt_launch(float *out, const float *x, const G53hMoeLayer *L, int *idx_out, float *w_out,
                      const int *idx_in, const float *w_in, char *buf, unsigned epoch)
{
    G53TiledArgs e;
    e.out = out; e.x = x; e.router = (const uint16_t *)L->router; e.bias = L->bias;
    e.experts = L->experts; e.shared = L->shared;
    e.score = (g53_u64 *)buf;
    e.act = (g53_u64 *)(buf + G53_DT_OFF_ACT + (epoch % G53_DT_ROT) * G53_DT_ACT_COPY);
    e.err = g53h_errblock() + 1; e.idx_out = idx_out; e.w_out = w_out; e.idx_in = idx_in; e.w_in = w_in;
    e.NE = L->n_experts; e.K = L->topk; e.norm_topk = L->norm_topk; e.epoch = epoch;
    e.spin = g53h_spin_limit(); e.routed_scale = L->routed_scale; e.limit = L->swiglu_limit; e.trace = g_dt_trace;
    e.nrouter = nullptr; e.nbias = nullptr; e.nscore = e.nchoice = nullptr;
    G53NextReq *nq = g53h_next_req();
    const int rows = (L->n_experts + g_dt_grid - 1) / g_dt_grid;
    /* the next layer's scores by spare waves: a bf16 router on this x, and at least two set-up
     * waves left (router rows + next rows + the routing wave + 2 <= the workgroup's waves) */
    if (nq->armed && nq->dt == 1 && nq->x == x && nq->NE == L->n_experts && nq->E == G53_DEC_E &&
        (idx_in ? 0 : rows) + rows + 3 <= G53_DT_NW) {
        float *nb = g53h_next_buf();
        e.nrouter = (const uint16_t *)nq->gate; e.nbias = nq->bias; e.nchoice = nb; e.nscore = nb + 1024;
        nq->armed = 0;
    }
    g53h_prof_mark(G53_PROF_START);
    if (L->tiled == 3)                 /* int4-tiled routed experts */
        hipLaunchKernelGGL(k_dec_tiled<true>, dim3(g_dt_grid), dim3(G53_DT_NT), 0, g53h_stream(), e);
    else
        hipLaunchKernelGGL(k_dec_tiled<false>, dim3(g_dt_grid), dim3(G53_DT_NT), 0, g53h_stream(), e);
    g53h_prof_mark(G53_PROF_FUSED);
}

/* Launch k_dec_tiled; returns 1 when the layer is not one it takes (the caller falls back). */
int g53h_decode_tiled(float *out, const float *x, const G53hMoeLayer *L, int *idx_out, float *w_out,
                      const int *idx_in, const float *w_in)
{
    if (!dt_takes(L, idx_in) || !dt_size_grid()) return 1;
    const size_t off_act = G53_DT_OFF_ACT, act_copy = G53_DT_ACT_COPY;
    if (!g_dt_buf) {
        const size_t bytes = off_act + G53_DT_ROT * act_copy;
        G53_TRY(hipMalloc(&g_dt_buf, bytes));
        G53_TRY(hipMemset(g_dt_buf, 0, bytes));
        G53_TRY(hipDeviceSynchronize());
        g_dt_buf_bytes = bytes;
        g_dt_epoch = 0;
    }
    if (++g_dt_epoch == 0) {                             /* wrapped: clear and start over */
        G53_TRY(hipStreamSynchronize(g53h_stream()));
        G53_TRY(hipMemset(g_dt_buf, 0, g_dt_buf_bytes));
        G53_TRY(hipDeviceSynchronize());
        g_dt_epoch = 1;
    }
    (void)off_act; (void)act_copy;
    dt_launch(out, x, L, idx_out, w_out, idx_in, w_in, (char *)g_dt_buf, g_dt_epoch);
    G53_LAUNCHED("k_dec_tiled");
    return 0;
}

/* ------------------------------------------------ the variant that allocates nothing ---- */
/* The same launch with its scratch in this file-scope array (zero at load; each device holds
 * its own copy until the process ends). Host code uses the per-device address from
 * hipGetSymbolAddress, never the array's name. Calls that overlap on one device race. */
static __device__ __align__(256) unsigned char scratch[G53_DT_SCRATCH];
#define G53_NA_MAXDEV 64
static void *g_na_ptr[G53_NA_MAXDEV];
static unsigned g_na_epoch[G53_NA_MAXDEV];

__global__ void k_na_clear(uint4 *p, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = make_uint4(0, 0, 0, 0);
}

/* Set-up, once per device with that device current (called by g53h_init). */
int g53_noalloc_setup(int device)
{
    if (device < 0 || device >= G53_NA_MAXDEV) return g53h_fail("g53h_moe_decode_noalloc: device %d", device);
    if (g_na_ptr[device]) return 0;
    void *p = nullptr;
    G53_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return g53h_fail("g53h_moe_decode_noalloc: no device address for the scratch array");
    g_na_ptr[device] = p;
    g_na_epoch[device] = 0;
    return 0;
}

extern "C" int g53h_moe_decode_noalloc(float *out_d, const float *x_d, const G53hMoeLayer *L, int *idx_d,
                                       float *w_d)
{
    const int dev = g53h_current_device();
    if (dev < 0 || dev >= G53_NA_MAXDEV || !g_na_ptr[dev])
        return g53h_fail("g53h_moe_decode_noalloc: call g53h_init on this device first");
    if (!L || !out_d || !x_d || !L->experts) return g53h_fail("g53h_moe_decode_noalloc: missing argument");
    if (L->n_experts < 1 || L->n_experts > G53_DEC_MAXNE)
        return g53h_fail("g53h_moe_decode_noalloc: %d routed experts, above the limit of %d", L->n_experts,
                         G53_DEC_MAXNE);
    if (L->topk < 1 || L->topk > G53_DEC_MAXK)
        return g53h_fail("g53h_moe_decode_noalloc: top-k %d, above the limit of %d", L->topk, G53_DEC_MAXK);
    if (L->tiled != 1 || !dt_takes(L, nullptr))
        return g53h_fail("g53h_moe_decode_noalloc: the layer must be octet-tiled with hidden %d, inter %d, "
                         "128-column blocks and a bf16 router", G53_DEC_E, G53_DEC_I);
    if (!dt_size_grid()) return g53h_fail("g53h_moe_decode_noalloc: the decode kernel does not fit this device");
    char *buf = (char *)g_na_ptr[dev];
    if (++g_na_epoch[dev] == 0) {                        /* wrapped: clear the tags, start over */
        const size_t n = G53_DT_SCRATCH / 16;
        hipLaunchKernelGGL(k_na_clear, dim3(1024), dim3(256), 0, g53h_stream(), (uint4 *)buf, n);
        G53_LAUNCHED("k_na_clear");
        g_na_epoch[dev] = 1;
    }
    dt_launch(out_d, x_d, L, idx_d, w_d, nullptr, nullptr, buf, g_na_epoch[dev]);
    G53_LAUNCHED("k_dec_tiled");
    return 0;
}
