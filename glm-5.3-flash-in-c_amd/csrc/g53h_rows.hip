/* g53h_rows.hip - the row-wave expert kernels (int4 experts and FP8 matrices of any geometry)
 * and the FP8 -> int4 quantiser, bit-exact with the reference:
 *
 *   k_rows_gateup   gate and up rows and their SwiGLU, k_rows_down the down rows, for the
 *                   (token, slot) pairs of a MoE layer: one one-wave workgroup per (token,
 *                   slot) and 4 rows of gate and up (8 rows of down). Every lane computes the
 *                   reference's sum of one column group of one row (the eight fp32 lanes, the
 *                   double tree, the tail) times its scale in double; the row's groups are then
 *                   added in order by one lane per row from LDS, as the reference's loop over
 *                   groups adds them (src/core/glm53f_ops.c:236-296 matmul_i4, :185-228
 *                   matmul_f8). Int4 matrices with 64-column groups keep the lane's 64
 *                   activations in registers and read each row's 32 bytes per lane in two
 *                   16-byte loads, so a wave streams whole rows. Octet-tiled FP8 matrices
 *                   (128-column blocks) take eight lanes per block, one per reference
 *                   accumulator, each reading its 16 codes as one 16-byte run of the tiled
 *                   unit. Anything else (row-major FP8, other group widths) reads per byte.
 *   k_i4_from_f8    one thread per (row, group of 64) (src/core/glm53f_ops.c:302-371).
 */
#include <hip/hip_runtime.h>
#include <math.h>

#include "g53h.h"
#include "g53h_core.h"
#include "g53h_kern.h"
#include "g53h_rowdot.h"
#include "g53h_runtime.h"

#define G53_RW_LD    65                 /* LDS row stride of the partials (doubles) */

typedef unsigned int g53_v4u __attribute__((ext_vector_type(4)));
#ifndef G53_RW_NT
#define G53_RW_NT 1
#endif
#if G53_RW_NT
#define G53_RW_W(p) __builtin_nontemporal_load(p)   /* weights are read once */
#else
#define G53_RW_W(p) (*(p))
#endif
#ifndef G53_RW_RB
#define G53_RW_RB 4                     /* octet-tiled rows whose 16-byte runs are loaded together */
#endif

/* One group of 64 int4 columns (32 bytes c0, c1) against 64 activations xr: the reference's
 * eight lanes stepping by 8 columns (src/core/glm53f_ops.c:247-282), then the double tree. */
__device__ __forceinline__ double g53_i4_group64(const g53_v4u &c0, const g53_v4u &c1, const float (&xr)[64])
{
    const uint32_t d[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < 8; k++) {               /* columns 8k .. 8k+7 are the nibbles of d[k] */
        /* even columns in the low nibble of each byte, odd ones in the high nibble: byte i of
         * the masked word becomes the low mantissa byte of 2^23 + nibble (one byte permute),
         * and subtracting 2^23 + 8 leaves the level nibble - 8, exact */
        const uint32_t lo = d[k] & 0x0f0f0f0fu, hi = (d[k] >> 4) & 0x0f0f0f0fu;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t sel = 0x070c0c00u | (uint32_t)i;       /* [byte i, 0, 0, 0x4b] */
            const float le = __builtin_bit_cast(float, __builtin_amdgcn_perm(0x4b000000u, lo, sel)) - 8388616.0f;
            const float lodd = __builtin_bit_cast(float, __builtin_amdgcn_perm(0x4b000000u, hi, sel)) - 8388616.0f;
            a[2 * i] = __builtin_fmaf(le, xr[8 * k + 2 * i], a[2 * i]);
            a[2 * i + 1] = __builtin_fmaf(lodd, xr[8 * k + 2 * i + 1], a[2 * i + 1]);
        }
    }
    return (((double)a[0] + a[4]) + ((double)a[2] + a[6])) + (((double)a[1] + a[5]) + ((double)a[3] + a[7]));
}

/* LDS written by some lanes of a wave and read by others of the same wave. */
__device__ __forceinline__ void g53_wave_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/* Lanes lo .. hi-1 add the partials of their buf rows (row = lane), n per row, in order onto acc. */
__device__ __forceinline__ double g53_chain(const double *buf, int n, int lane, int lo, int hi, double acc)
{
    g53_wave_sync();
    if (lane >= lo && lane < hi)
        for (int k = 0; k < n; k++) acc = acc + buf[lane * G53_RW_LD + k];
    g53_wave_sync();
    return acc;
}

/* An int4 matrix the register path takes: 64-column groups, 3 to 64 of them, 16-byte aligned. */
__device__ __forceinline__ bool g53_i4_fast(const G53hMat &m, const float *xt)
{
    return (m.flags & G53H_MAT_I4) && m.bc == 64 && m.cols == 64 * m.scols && m.scols >= 3 && m.scols <= 64 &&
           ((uintptr_t)m.w & 15) == 0 && ((uintptr_t)xt & 15) == 0;
}

/* Lanes per row of the register path: a power of two >= the group count, and >= 64 / nr so
 * that the 64 / lanes rows of one step fit in the nr rows of a pass. */
__device__ __forceinline__ int g53_lpr(int ng, int nr)
{
    const int l = ng > 32 ? 64 : (ng > 16 ? 32 : (ng > 8 ? 16 : (ng > 4 ? 8 : 4)));
    return l * nr >= 64 ? l : 64 / nr;
}

/* The lane's 64 activations of group g (zeros for g >= ng). */
__device__ __forceinline__ void g53_x_group(float (&xr)[64], const float *xt, int g, int ng)
{
    if (g < ng) {
        const float4 *xv = (const float4 *)(xt + g * 64);
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const float4 v = xv[k];
            xr[4 * k] = v.x; xr[4 * k + 1] = v.y; xr[4 * k + 2] = v.z; xr[4 * k + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < 64; k++) xr[k] = 0.0f;
    }
}

/* Rows row0 .. row0+NR-1 (those below `rows`) of matrix m times xt, as the reference sums them
 * (glm53f_mm per row, in double): the partials go to buf rows off .. off+NR-1 and lane off + i
 * adds row row0 + i onto acc, which it returns (other lanes return acc unchanged). The whole
 * wave calls it; the path depends on m only. */
template <int NR>
__device__ __forceinline__ double g53_pass(const G53hMat &m, const float *__restrict__ xt, int row0, int rows,
                                           double *buf, int off, int lane, double acc)
{
    const bool i4 = (m.flags & G53H_MAT_I4) != 0;
    if (!i4 && (m.flags & G53H_MAT_TILED)) {
        /* octet-tiled FP8: 8 lanes per 128-column block, lane l holding the reference's
         * accumulator l (its 16 codes are one 16-byte run of the tiled unit), 8 blocks per
         * step and up to 32 blocks per pass with their activations in registers; the eight
         * accumulators are joined by the reference's tree across the lanes */
        const int nb = m.scols, j = lane >> 3, l = lane & 7;
        const int run = ((l & 1) << 2) | (l & 2) | (l >> 2);       /* the run holding accumulator l */
        for (int c0 = 0; c0 < nb; c0 += 32) {
            const int nbc = nb - c0 < 32 ? nb - c0 : 32, nst = (nbc + 7) >> 3;
            float xr[64];
#pragma unroll
            for (int st = 0; st < 4; st++)
#pragma unroll
                for (int k = 0; k < 16; k++) {
                    const int b = st * 8 + j;
                    xr[st * 16 + k] = b < nbc ? xt[(c0 + b) * 128 + l + 8 * k] : 0.0f;
                }
            constexpr int RB = NR < G53_RW_RB ? NR : G53_RW_RB;  /* rows whose runs are in flight */
            for (int r4 = 0; r4 < NR; r4 += RB) {
                g53_v4u c[RB][4];
#pragma unroll
                for (int i = 0; i < RB; i++)
#pragma unroll
                    for (int st = 0; st < 4; st++) {
                        const int r = row0 + r4 + i, b = st * 8 + j;
                        if (st < nst && b < nbc && r < rows)
                            c[i][st] = G53_RW_W((const g53_v4u *)(m.w + ((size_t)(r >> 3) * nb + c0 + b) * 1024 +
                                                                  (r & 7) * 128 + run * 16));
                        else
                            c[i][st] = g53_v4u{0, 0, 0, 0};
                    }
#pragma unroll
                for (int i = 0; i < RB; i++) {
                    const int r = row0 + r4 + i;
                    const float *srow = m.s + (size_t)(r / m.br) * nb + c0;
#pragma unroll
                    for (int st = 0; st < 4; st++) {
                        const int b = st * 8 + j;
                        if (st < nst && b < nbc && r < rows) {               /* uniform across 8 lanes */
                            const float *xs = xr + st * 16;
                            float a = 0.0f;
#pragma unroll
                            for (int q = 0; q < 4; q++) {  /* codes 4q .. 4q+3, in column order */
                                const int d = (int)c[i][st][q];
                                a = __builtin_fmaf(__builtin_amdgcn_cvt_f32_fp8(d, 0), xs[4 * q], a);
                                a = __builtin_fmaf(__builtin_amdgcn_cvt_f32_fp8(d, 1), xs[4 * q + 1], a);
                                a = __builtin_fmaf(__builtin_amdgcn_cvt_f32_fp8(d, 2), xs[4 * q + 2], a);
                                a = __builtin_fmaf(__builtin_amdgcn_cvt_f32_fp8(d, 3), xs[4 * q + 3], a);
                            }
                            /* ((a0 + a4) + (a2 + a6)) + ((a1 + a5) + (a3 + a7)), each pair in double */
                            double v = (double)a;
                            v = v + __shfl_xor(v, 4, 8);
                            v = v + __shfl_xor(v, 2, 8);
                            v = v + __shfl_xor(v, 1, 8);
                            if (l == 0) buf[(off + r4 + i) * G53_RW_LD + b] = v * (double)srow[b];
                        }
                    }
                }
            }
            acc = g53_chain(buf, nbc, lane, off, off + NR, acc);
        }
        return acc;
    }
    if (g53_i4_fast(m, xt)) {
        /* lpr lanes per row, 64 / lpr rows per step; every row's 32 bytes per lane are loaded
         * before any is used */
        const int ng = m.scols, lpr = g53_lpr(ng, NR);
        const int rps = 64 / lpr, nst = NR / rps, g = lane & (lpr - 1), sub = lane / lpr;
        float xr[64];
        g53_x_group(xr, xt, g, ng);
        const size_t rb = (size_t)m.cols / 2;
        g53_v4u c0[NR], c1[NR];
        float stp[NR];
#pragma unroll
        for (int st = 0; st < NR; st++) {
            const int r = row0 + st * rps + sub;
            if (st < nst && g < ng && r < rows) {
                const g53_v4u *w = (const g53_v4u *)(m.w + (size_t)r * rb + (size_t)g * 32);
                c0[st] = G53_RW_W(w);
                c1[st] = G53_RW_W(w + 1);
                stp[st] = m.s[(size_t)r * ng + g];
            } else {
                c0[st] = g53_v4u{0, 0, 0, 0};
                c1[st] = g53_v4u{0, 0, 0, 0};
                stp[st] = 0.0f;
            }
        }
#pragma unroll
        for (int st = 0; st < NR; st++) {
            const int rl = st * rps + sub;
            if (st < nst && g < ng && row0 + rl < rows)
                buf[(off + rl) * G53_RW_LD + g] = g53_i4_group64(c0[st], c1[st], xr) * (double)stp[st];
        }
        return g53_chain(buf, ng, lane, off, off + NR, acc);
    }
    /* any geometry: lane b takes column block (group) c0 + b of one row per step */
    const int nb = m.scols;
    for (int c0 = 0; c0 < nb; c0 += 64) {
        const int b = c0 + lane, j0 = b * m.bc, j1 = j0 + m.bc < m.cols ? j0 + m.bc : m.cols;
        for (int rl = 0; rl < NR; rl++) {
            const int r = row0 + rl;
            if (b < nb && r < rows) {
                double p;
                if (i4) {
                    p = g53_group_dot_i4(m.w + (size_t)r * (m.cols / 2), xt, j0, j1) * (double)m.s[(size_t)r * nb + b];
                } else {
                    p = g53_block_dot(m.w + (size_t)r * m.cols, xt, j0, j1) *
                        (double)m.s[(size_t)(r / m.br) * nb + b];
                }
                buf[(off + rl) * G53_RW_LD + lane] = p;
            }
        }
        acc = g53_chain(buf, nb - c0 < 64 ? nb - c0 : 64, lane, off, off + NR, acc);
    }
    return acc;
}

/* A usable octet-tiled matrix: 128-column blocks and whole row octets (the tiled format's
 * definition); anything else marked tiled is not read. */
__device__ __forceinline__ bool g53_rows_ok(const G53hMat &m)
{
    if (!(m.flags & G53H_MAT_TILED) || (m.flags & G53H_MAT_I4)) return true;
    return m.bc == 128 && m.cols == 128 * m.scols && (m.rows & 7) == 0 && ((uintptr_t)m.w & 15) == 0;
}

/* Sizes measured on MI355X (config-2 int4 decode): one wave per workgroup, 4 gate rows (and 4
 * up rows) or 8 down rows per wave keep the kernels at 3 waves per SIMD for the down rows and 2
 * for gate/up; 8-wave workgroups, or 8 gate / 16 down rows per wave, were slower. */
#ifndef G53_RW_NW
#define G53_RW_NW 1                     /* waves per workgroup, each with rows of its own */
#endif
#ifndef G53_GU_ROWS
#define G53_GU_ROWS 4                   /* gate rows (and as many up rows) per wave */
#endif
#ifndef G53_DN_ROWS
#define G53_DN_ROWS 8                   /* down rows per wave                      */
#endif

/* blockIdx.y = t * (nslots + 1) + r -> (token t, slot s, half h): r = 0 and 1 are the two halves
 * of the last slot, r >= 2 slot nslots - r, whole. The last slot is the shared expert when there
 * is one (FP8, twice the bytes of an int4 expert): dispatched first, it overlaps the routed
 * experts instead of trailing them, and octet-tiled it is split over two workgroups so that
 * no workgroup carries more bytes than an int4 one. Any other matrix takes half 0 whole (its
 * half 1 workgroup exits at once). */
__device__ __forceinline__ void g53_rows_slot(int nslots, int &t, int &s, int &h)
{
    const int per = nslots + 1, r = (int)(blockIdx.y % per);
    t = (int)(blockIdx.y / per);
    s = r <= 1 ? nslots - 1 : nslots - r;
    h = r <= 1 ? r : 0;
}

__device__ __forceinline__ bool g53_split(const G53hMat &m)
{
    return !(m.flags & G53H_MAT_I4) && (m.flags & G53H_MAT_TILED);
}

/* Gate, up and SwiGLU for (token, slot) of descriptors slots [T][nslots] times x [T][E]:
 * act [T][nslots][I] = swiglu_clamp(gate row, up row). One wave per G53_GU_ROWS rows of both
 * matrices (half as many for a split octet-tiled slot), lanes 0-3 summing the gate rows and 4-7 the
 * up rows; with int4 experts every load of both matrices is issued before any is used. A
 * descriptor with gate.w NULL is absent from this call (nothing written) unless marked dropped
 * (zeros). */
__global__ void __launch_bounds__(64 * G53_RW_NW)
k_rows_gateup(float *__restrict__ act, const float *__restrict__ x, int nslots, const G53hExpert *__restrict__ slots,
              int I, int E, float limit)
{
    __shared__ double bufs[G53_RW_NW][2 * G53_GU_ROWS * G53_RW_LD];
    int t, s, h;
    g53_rows_slot(nslots, t, s, h);
    const int ts = t * nslots + s, lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    double *buf = bufs[wv];
    const G53hExpert &e = slots[ts];
    const bool split = e.gate.w && g53_split(e.gate) && g53_split(e.up);
    if (h && !split) return;
    const int nr = split ? G53_GU_ROWS / 2 : G53_GU_ROWS, row0 = (blockIdx.x * G53_RW_NW + wv) * G53_GU_ROWS + h * nr;
    if (row0 >= I) return;
    float *at = act + (size_t)ts * I;
    const bool write = lane < nr && row0 + lane < I;
    if (!e.gate.w) {
        if ((e.gate.flags & G53H_MAT_DROPPED) && write) at[row0 + lane] = 0.0f;
        return;
    }
    const G53hMat g = e.gate, u = e.up;
    if (!g53_rows_ok(g) || !g53_rows_ok(u)) {                   /* malformed: NaN, not misread */
        if (write) at[row0 + lane] = __builtin_nanf("");
        return;
    }
    const float *xt = x + (size_t)t * E;
    double acc = 0.0;
    if (g53_i4_fast(g, xt) && g53_i4_fast(u, xt) && g.scols == u.scols) {
        const int ng = g.scols, lpr = g53_lpr(ng, G53_GU_ROWS);
        const int rps = 64 / lpr, nst = G53_GU_ROWS / rps, gi = lane & (lpr - 1), sub = lane / lpr;
        const size_t rb = (size_t)g.cols / 2;
        g53_v4u c0[2 * G53_GU_ROWS], c1[2 * G53_GU_ROWS];
        float stp[2 * G53_GU_ROWS];
#pragma unroll
        for (int k = 0; k < 2 * G53_GU_ROWS; k++) {               /* gate rows, then up rows */
            const G53hMat &m = k < G53_GU_ROWS ? g : u;
            const int st = k % G53_GU_ROWS, r = row0 + st * rps + sub;
            if (st < nst && gi < ng && r < I) {
                const g53_v4u *w = (const g53_v4u *)(m.w + (size_t)r * rb + (size_t)gi * 32);
                c0[k] = G53_RW_W(w);
                c1[k] = G53_RW_W(w + 1);
                stp[k] = m.s[(size_t)r * ng + gi];
            } else {
                c0[k] = g53_v4u{0, 0, 0, 0};
                c1[k] = g53_v4u{0, 0, 0, 0};
                stp[k] = 0.0f;
            }
        }
        float xr[64];
        g53_x_group(xr, xt, gi, ng);
#pragma unroll
        for (int k = 0; k < 2 * G53_GU_ROWS; k++) {
            const int st = k % G53_GU_ROWS, rl = st * rps + sub;
            if (st < nst && gi < ng && row0 + rl < I)
                buf[((k < G53_GU_ROWS ? 0 : G53_GU_ROWS) + rl) * G53_RW_LD + gi] =
                    g53_i4_group64(c0[k], c1[k], xr) * (double)stp[k];
        }
        acc = g53_chain(buf, ng, lane, 0, 2 * G53_GU_ROWS, acc);
    } else if (split) {
        acc = g53_pass<G53_GU_ROWS / 2>(g, xt, row0, I, buf, 0, lane, acc);
        acc = g53_pass<G53_GU_ROWS / 2>(u, xt, row0, I, buf, G53_GU_ROWS, lane, acc);
    } else {
        acc = g53_pass<G53_GU_ROWS>(g, xt, row0, I, buf, 0, lane, acc);
        acc = g53_pass<G53_GU_ROWS>(u, xt, row0, I, buf, G53_GU_ROWS, lane, acc);
    }
    const double au = __shfl_down(acc, G53_GU_ROWS);
    if (write) at[row0 + lane] = g53_swiglu1((float)acc, (float)au, limit);
}

/* Down: y [T][nslots][E] = down(slot) . act [T][nslots][I], one wave per G53_DN_ROWS rows (half for a split
 * octet-tiled slot; the slot order of k_rows_gateup). */
__global__ void __launch_bounds__(64 * G53_RW_NW)
k_rows_down(float *__restrict__ y, const float *__restrict__ act, int nslots, const G53hExpert *__restrict__ slots,
            int E, int I)
{
    __shared__ double bufs[G53_RW_NW][G53_DN_ROWS * G53_RW_LD];
    int t, s, h;
    g53_rows_slot(nslots, t, s, h);
    const int ts = t * nslots + s, lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    double *buf = bufs[wv];
    const G53hExpert &e = slots[ts];
    const bool split = e.gate.w && g53_split(e.down);
    if (h && !split) return;
    const int nr = split ? G53_DN_ROWS / 2 : G53_DN_ROWS, row0 = (blockIdx.x * G53_RW_NW + wv) * G53_DN_ROWS + h * nr;
    if (row0 >= E) return;
    float *yt = y + (size_t)ts * E;
    const bool write = lane < nr && row0 + lane < E;
    if (!e.gate.w) {
        if ((e.gate.flags & G53H_MAT_DROPPED) && write) yt[row0 + lane] = 0.0f;
        return;
    }
    const G53hMat d = e.down;
    if (!g53_rows_ok(d)) {
        if (write) yt[row0 + lane] = __builtin_nanf("");
        return;
    }
    const float *xt = act + (size_t)ts * I;
    const double a = split ? g53_pass<G53_DN_ROWS / 2>(d, xt, row0, E, buf, 0, lane, 0.0)
                           : g53_pass<G53_DN_ROWS>(d, xt, row0, E, buf, 0, lane, 0.0);
    if (write) yt[row0 + lane] = (float)a;
}

int g53h_rows_layer(float *contrib, float *act, const float *x, int T, int nslots, const G53hExpert *slots, int E,
                    int I, float limit)
{
    if (T <= 0 || nslots <= 0) return 0;
    if ((long)T * (nslots + 1) > 65535) return g53h_fail("g53h_rows_layer: %d (token, slot) pairs", T * nslots);
    const unsigned ny = (unsigned)(T * (nslots + 1));
    const int gu = G53_GU_ROWS * G53_RW_NW, dn = G53_DN_ROWS * G53_RW_NW;
    hipLaunchKernelGGL(k_rows_gateup, dim3((unsigned)((I + gu - 1) / gu), ny), dim3(64 * G53_RW_NW), 0,
                       g53h_stream(), act, x, nslots, slots, I, E, limit);
    G53_LAUNCHED("k_rows_gateup");
    hipLaunchKernelGGL(k_rows_down, dim3((unsigned)((E + dn - 1) / dn), ny), dim3(64 * G53_RW_NW), 0,
                       g53h_stream(), contrib, act, nslots, slots, E, I);
    G53_LAUNCHED("k_rows_down");
    return 0;
}

/* ------------------------------------------------------------------ quantiser ---- */
__global__ void k_i4_from_f8(uint8_t *__restrict__ q, float *__restrict__ steps, G53hMat src)
{
    const int groups = src.cols / 64;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)src.rows * groups) return;
    const int o = (int)(i / groups), g = (int)(i % groups), j0 = g * 64;
    const uint8_t *row = src.w + (size_t)o * src.cols;
    const float *srow = src.s + (size_t)(o / src.br) * src.scols;
    const bool aligned = src.bc % 64 == 0;            /* one FP8 scale for the group */
    const float bs = srow[j0 / src.bc];
    /* the group's values are decoded twice (maximum, then levels) rather than kept */
    float amax = 0.0f;
    for (int j = 0; j < 64; j++) {
        const float w = g53_e4m3_to_f32(row[j0 + j]) * (aligned ? 1.0f : srow[(j0 + j) / src.bc]);
        const float a = w < 0.0f ? -w : w;
        if (a > amax) amax = a;
    }
    float step = (aligned ? amax * bs : amax) / 7.0f;
    if (!(step > 1e-30f)) step = 1e-30f;
    steps[(size_t)o * groups + g] = step;
    const float inv = amax > 0.0f ? 7.0f / amax : 0.0f;
    const float mul = aligned ? inv : 1.0f / step;
    uint8_t *dst = q + (size_t)o * (src.cols / 2) + j0 / 2;
    for (int j = 0; j < 64; j += 2) {
        const float v0 = g53_e4m3_to_f32(row[j0 + j]) * (aligned ? 1.0f : srow[(j0 + j) / src.bc]);
        const float v1 = g53_e4m3_to_f32(row[j0 + j + 1]) * (aligned ? 1.0f : srow[(j0 + j + 1) / src.bc]);
        const float f0 = v0 * mul, f1 = v1 * mul;
        int l0 = f0 == f0 ? (int)rintf(f0 < -16.0f ? -16.0f : (f0 > 16.0f ? 16.0f : f0)) : 0;
        int l1 = f1 == f1 ? (int)rintf(f1 < -16.0f ? -16.0f : (f1 > 16.0f ? 16.0f : f1)) : 0;
        l0 = l0 < -8 ? -8 : (l0 > 7 ? 7 : l0);
        l1 = l1 < -8 ? -8 : (l1 > 7 ? 7 : l1);
        dst[j >> 1] = (uint8_t)((l0 + 8) | ((l1 + 8) << 4));
    }
}

extern "C" int g53h_i4_from_f8(uint8_t *q, float *steps, const G53hMat *m)
{
    if (g53h_ready()) return -1;
    return g53h_i4_from_f8_on(q, steps, m, g53h_stream());
}

int g53h_i4_from_f8_on(uint8_t *q, float *steps, const G53hMat *m, hipStream_t stream)
{
    if (!m || !m->w || !m->s || !q || !steps) return g53h_fail("g53h_i4_from_f8: unbound matrix");
    if ((m->flags & (G53H_MAT_I4 | G53H_MAT_TILED)) || m->rows <= 0 || m->cols <= 0 || m->cols % 64 ||
        m->br <= 0 || m->bc <= 0 || m->scols != (m->cols + m->bc - 1) / m->bc)
        return g53h_fail("g53h_i4_from_f8: needs a row-major FP8 matrix with columns a multiple of 64 (%dx%d, "
                         "block %dx%d, scols %d, flags %d)", m->rows, m->cols, m->br, m->bc, m->scols, m->flags);
    const long n = (long)m->rows * (m->cols / 64);
    hipLaunchKernelGGL(k_i4_from_f8, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, q, steps, *m);
    G53_LAUNCHED("k_i4_from_f8");
    return 0;
}
