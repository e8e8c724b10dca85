/* g53h_rows.hip - the row-wave expert kernels (int4 experts and FP8 matrices of any geometry)
 * and the FP8 -> int4 quantiser, bit-exact with the reference:
 *
 *   k_slot_rows     y = M . x for the (token, slot) pairs of a MoE layer, one workgroup per
 *                   (token, slot) and 64 rows, one wave per 16 rows. Every lane computes the
 *                   reference's sum of one column group of one row (the eight fp32 lanes, the
 *                   double tree, the tail) times its scale in double; the row's groups are then
 *                   added in order by one lane per row from LDS, as the reference's loop over
 *                   groups adds them (src/core/glm53f_ops.c:236-296 matmul_i4, :185-228
 *                   matmul_f8). Int4 matrices with 64-column groups keep the lane's 64
 *                   activations in registers and read each row's 32 bytes per lane in two
 *                   16-byte loads, so a wave streams whole rows; anything else (FP8, other
 *                   group widths) reads per byte.
 *   k_i4_from_f8    one thread per (row, group of 64) (src/core/glm53f_ops.c:302-371).
 */
#include <hip/hip_runtime.h>
#include <math.h>

#include "g53h.h"
#include "g53h_core.h"
#include "g53h_kern.h"
#include "g53h_rowdot.h"
#include "g53h_runtime.h"

#define G53_RW_ROWS  16                 /* rows per wave                          */
#define G53_RW_WAVES 4                  /* waves per workgroup                    */
#define G53_RW_LD    65                 /* LDS row stride of the partials (doubles) */

typedef unsigned int g53_v4u __attribute__((ext_vector_type(4)));

/* One group of 64 int4 columns (32 bytes c[0..1]) against 64 activations xr: the reference's
 * eight lanes stepping by 8 columns, then the double tree. */
__device__ __forceinline__ double g53_i4_group64(const g53_v4u &c0, const g53_v4u &c1, const float (&xr)[64])
{
    const uint32_t d[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < 8; k++)                  /* columns 8k .. 8k+7 are the nibbles of d[k] */
#pragma unroll
        for (int l = 0; l < 8; l++)
            a[l] = __builtin_fmaf((float)((int)((d[k] >> (4 * l)) & 15u) - 8), xr[8 * k + l], a[l]);
    return (((double)a[0] + a[4]) + ((double)a[2] + a[6])) + (((double)a[1] + a[5]) + ((double)a[3] + a[7]));
}

/* The (token, slot) pair of blockIdx.y multiplies matrix `which` (0 gate, 1 up, 2 down) of its
 * descriptor slots[t * nslots + s] with x (per token, or per (token, slot) when x_per_slot) into
 * y [T][nslots][rows]. A descriptor with gate.w NULL is absent from this call (nothing written)
 * unless marked dropped (zeros written). */
__global__ void __launch_bounds__(64 * G53_RW_WAVES)
k_slot_rows(float *__restrict__ y, const float *__restrict__ x, int nslots, const G53hExpert *__restrict__ slots,
            int which, int rows, int cols, int x_per_slot)
{
    __shared__ double part[G53_RW_WAVES][G53_RW_ROWS * G53_RW_LD];
    const int ts = blockIdx.y, s = ts % nslots, t = ts / nslots;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * G53_RW_WAVES + wave) * G53_RW_ROWS;
    const G53hExpert &e = slots[ts];
    const G53hMat m = which == 0 ? e.gate : (which == 1 ? e.up : e.down);
    float *yt = y + (size_t)ts * rows;
    if (!e.gate.w) {
        if ((e.gate.flags & G53H_MAT_DROPPED) && lane < G53_RW_ROWS && row0 + lane < rows) yt[row0 + lane] = 0.0f;
        return;
    }
    const float *xt = x + ((size_t)t * (x_per_slot ? nslots : 1) + (x_per_slot ? s : 0)) * cols;
    double *buf = part[wave];
    double acc = 0.0;                            /* lanes < 16: the row row0 + lane */
    const bool i4 = (m.flags & G53H_MAT_I4) != 0;
    const bool fast = i4 && m.bc == 64 && m.cols == 64 * m.scols && m.scols >= 3 && m.scols <= 64 &&
                      ((uintptr_t)m.w & 15) == 0 && ((uintptr_t)xt & 15) == 0;
    if (fast) {
        /* lpr lanes per row (a power of two >= the group count), 64 / lpr rows per step */
        const int ng = m.scols;
        const int lpr = ng > 32 ? 64 : (ng > 16 ? 32 : (ng > 8 ? 16 : (ng > 4 ? 8 : 4)));
        const int rps = 64 / lpr, g = lane & (lpr - 1), sub = lane / lpr;
        float xr[64];
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
        const size_t rb = (size_t)m.cols / 2;
        for (int st = 0; st < G53_RW_ROWS; st += rps) {
            const int rl = st + sub, r = row0 + rl;
            if (g < ng && r < rows) {
                const g53_v4u *w = (const g53_v4u *)(m.w + (size_t)r * rb + (size_t)g * 32);
                const g53_v4u c0 = __builtin_nontemporal_load(w), c1 = __builtin_nontemporal_load(w + 1);
                const float step = m.s[(size_t)r * ng + g];
                buf[rl * G53_RW_LD + g] = g53_i4_group64(c0, c1, xr) * (double)step;
            }
        }
        __syncthreads();
        if (lane < G53_RW_ROWS)
            for (int k = 0; k < ng; k++) acc = acc + buf[lane * G53_RW_LD + k];
    } else {
        /* any geometry: lane b takes column block (group) c0 + b of one row per step */
        const int nb = m.scols;
        for (int c0 = 0; c0 < nb; c0 += 64) {
            const int b = c0 + lane, j0 = b * m.bc, j1 = j0 + m.bc < m.cols ? j0 + m.bc : m.cols;
            for (int rl = 0; rl < G53_RW_ROWS; rl++) {
                const int r = row0 + rl;
                if (b < nb && r < rows) {
                    double p;
                    if (i4) {
                        p = g53_group_dot_i4(m.w + (size_t)r * (m.cols / 2), xt, j0, j1) *
                            (double)m.s[(size_t)r * nb + b];
                    } else {
                        p = g53_block_dot(m.w + (size_t)r * m.cols, xt, j0, j1) *
                            (double)m.s[(size_t)(r / m.br) * nb + b];
                    }
                    buf[rl * G53_RW_LD + lane] = p;
                }
            }
            __syncthreads();
            const int n = nb - c0 < 64 ? nb - c0 : 64;
            if (lane < G53_RW_ROWS)
                for (int k = 0; k < n; k++) acc = acc + buf[lane * G53_RW_LD + k];
            __syncthreads();
        }
    }
    if (lane < G53_RW_ROWS && row0 + lane < rows) yt[row0 + lane] = (float)acc;
}

int g53h_slot_rows(float *y, const float *x, int T, int nslots, const G53hExpert *slots, int which, int rows,
                   int cols, int x_per_slot)
{
    if (T <= 0 || nslots <= 0 || rows <= 0) return 0;
    if ((long)T * nslots > 65535) return g53h_fail("g53h_slot_rows: %d (token, slot) pairs", T * nslots);
    const int per_wg = G53_RW_ROWS * G53_RW_WAVES;
    hipLaunchKernelGGL(k_slot_rows, dim3((unsigned)((rows + per_wg - 1) / per_wg), (unsigned)(T * nslots)),
                       dim3(64 * G53_RW_WAVES), 0, g53h_stream(), y, x, nslots, slots, which, rows, cols, x_per_slot);
    G53_LAUNCHED("k_slot_rows");
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
