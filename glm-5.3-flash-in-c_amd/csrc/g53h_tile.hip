/* g53h_tile.hip - conversion of FP8 code matrices between the row-major layout of the
 * checkpoint (src/io/glm53f_load.c:171-179 keeps experts row-major) and the octet-tiled layout
 * the decode kernel streams (include/g53h.h, G53H_MAT_TILED).
 *
 * Output-major: thread q writes the 16-byte run q of the tiled matrix, whose bytes come from one
 * row's 128-column block (16 codes 8 columns apart). The source block is read once per run
 * through the caches; the conversion runs once per expert, when it enters HBM. */
#include <hip/hip_runtime.h>
#include <string.h>

#include "g53h.h"
#include "g53h_runtime.h"

namespace {

/* Run q of the tiled matrix: unit q / 64 (row octet u / nb, block u % nb), row (q % 64) / 8 of
 * the octet, run p = q % 8 holding accumulator a = g53h_tile_acc(p). */
__host__ __device__ inline void g53_tile_run(int q, int nb, int &row, int &col0)
{
    const int u = q >> 6, l = q & 63, p = l & 7;
    row = (u / nb) * 8 + (l >> 3);
    col0 = (u % nb) * 128 + (((p & 1) << 2) | (p & 2) | (p >> 2));   /* g53h_tile_acc(p) */
}

__global__ void __launch_bounds__(256) k_tile_f8(uint8_t *__restrict__ dst, const uint8_t *__restrict__ src,
                                                 int cols, long nrun)
{
    const long q = (long)blockIdx.x * 256 + threadIdx.x;
    if (q >= nrun) return;
    int row, c0;
    g53_tile_run((int)q, cols / 128, row, c0);
    const uint8_t *s = src + (size_t)row * cols + c0;
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; k++)
        w[k] = (uint32_t)s[32 * k] | ((uint32_t)s[32 * k + 8] << 8) | ((uint32_t)s[32 * k + 16] << 16) |
               ((uint32_t)s[32 * k + 24] << 24);
    *(uint4 *)(dst + 16 * q) = make_uint4(w[0], w[1], w[2], w[3]);
}

__global__ void __launch_bounds__(256) k_untile_f8(uint8_t *__restrict__ dst, const uint8_t *__restrict__ src,
                                                   int cols, long nrun)
{
    const long q = (long)blockIdx.x * 256 + threadIdx.x;
    if (q >= nrun) return;
    int row, c0;
    g53_tile_run((int)q, cols / 128, row, c0);
    const uint4 v = *(const uint4 *)(src + 16 * q);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint8_t *d = dst + (size_t)row * cols + c0;
#pragma unroll
    for (int i = 0; i < 16; i++) d[8 * i] = (uint8_t)(w[i >> 2] >> (8 * (i & 3)));
}

int g53_tile_shape(int rows, int cols)
{
    if (rows <= 0 || cols <= 0 || rows % 8 || cols % 128)
        return g53h_fail("g53h_tile_f8: a %d x %d matrix cannot be octet-tiled (rows a multiple of 8, "
                         "columns of 128)", rows, cols);
    return 0;
}

} /* namespace */

int g53h_tile_f8_on(uint8_t *dst_d, const uint8_t *src_d, int rows, int cols, hipStream_t s)
{
    if (g53h_ready() || g53_tile_shape(rows, cols)) return -1;
    if (dst_d == src_d) return g53h_fail("g53h_tile_f8: in-place conversion is not supported");
    const long nrun = (long)rows * cols / 16;
    hipLaunchKernelGGL(k_tile_f8, dim3((unsigned)((nrun + 255) / 256)), dim3(256), 0, s, dst_d, src_d, cols, nrun);
    G53_LAUNCHED("k_tile_f8");
    return 0;
}

extern "C" int g53h_tile_f8(uint8_t *dst_d, const uint8_t *src_d, int rows, int cols)
{
    if (g53h_ready()) return -1;
    return g53h_tile_f8_on(dst_d, src_d, rows, cols, g53h_stream());
}

extern "C" int g53h_untile_f8(uint8_t *dst_d, const uint8_t *src_d, int rows, int cols)
{
    if (g53h_ready() || g53_tile_shape(rows, cols)) return -1;
    if (dst_d == src_d) return g53h_fail("g53h_untile_f8: in-place conversion is not supported");
    const long nrun = (long)rows * cols / 16;
    hipLaunchKernelGGL(k_untile_f8, dim3((unsigned)((nrun + 255) / 256)), dim3(256), 0, g53h_stream(), dst_d,
                       src_d, cols, nrun);
    G53_LAUNCHED("k_untile_f8");
    return 0;
}

extern "C" int g53h_tile_f8_host(uint8_t *dst, const uint8_t *src, int rows, int cols, int inverse)
{
    if (rows <= 0 || cols <= 0 || rows % 8 || cols % 128 || dst == src) return -1;
    const long nrun = (long)rows * cols / 16;
    for (long q = 0; q < nrun; q++) {
        int row, c0;
        g53_tile_run((int)q, cols / 128, row, c0);
        for (int i = 0; i < 16; i++) {
            if (inverse) dst[(size_t)row * cols + c0 + 8 * i] = src[16 * q + i];
            else dst[16 * q + i] = src[(size_t)row * cols + c0 + 8 * i];
        }
    }
    return 0;
}

/* ---------------------------------------------------------- MFMA-tiled layout ---- */
/* The same 1 KB units (8 rows x 128 columns at ((r / 8) * (cols / 128) + c / 128) KB), with the
 * bytes inside a unit in the order the matrix cores take them (G53H_MAT_MTILED): column
 * c = 32 g + 16 i + j of unit row m sits at i * 512 + (8 g + m) * 16 + j. Sixteen-byte piece q
 * of a unit is (i, g, m) = (q / 32, (q / 8) % 4, q % 8). */
namespace {

__host__ __device__ inline void g53_mtile_piece(long q, int nb, int &row, int &col0)
{
    const long u = q >> 6;
    const int pc = (int)(q & 63), i = pc >> 5, g = (pc >> 3) & 3, m = pc & 7;
    row = (int)(u / nb) * 8 + m;
    col0 = (int)(u % nb) * 128 + 32 * g + 16 * i;
}

__global__ void __launch_bounds__(256) k_mtile_f8(uint8_t *__restrict__ dst, const uint8_t *__restrict__ src,
                                                  int cols, long npc, int inverse)
{
    const long q = (long)blockIdx.x * 256 + threadIdx.x;
    if (q >= npc) return;
    int row, c0;
    g53_mtile_piece(q, cols / 128, row, c0);
    uint4 *rm = (uint4 *)(inverse ? dst : src) + ((size_t)row * cols + c0) / 16;
    uint4 *tl = (uint4 *)(inverse ? src : dst) + q;
    if (inverse) *rm = *tl;
    else *tl = *rm;
}

/* Dword q of an int4-tiled matrix (G53H_MAT_I4T): unit u = q / 256 (row octet u / nb, 256-column
 * block u % nb), row m = (q % 256) / 32 of the octet, lane run p = (q % 32) / 4 (accumulator
 * g53h_tile_acc(p)), group g = q % 4 of the block. Its nibble i (low nibble first) is the level of
 * column block * 256 + 64 g + acc + 8 i. */
__host__ __device__ inline void g53_i4tile_dword(long q, int nb, int &row, int &col0)
{
    const long u = q >> 8;
    const int l = (int)(q & 255), m = l >> 5, p = (l >> 2) & 7, g = l & 3;
    row = (int)(u / nb) * 8 + m;
    col0 = (int)(u % nb) * 256 + 64 * g + (((p & 1) << 2) | (p & 2) | (p >> 2));
}

/* The level of column c of a row-major int4 row (low nibble = even column). */
__host__ __device__ inline unsigned g53_i4_get(const uint8_t *row, int c) { return (row[c >> 1] >> (4 * (c & 1))) & 15u; }

__global__ void __launch_bounds__(256) k_tile_i4(uint8_t *__restrict__ dst, const uint8_t *__restrict__ src,
                                                 int cols, long ndw, int inverse)
{
    const long q = (long)blockIdx.x * 256 + threadIdx.x;
    if (q >= ndw) return;
    int row, c0;
    g53_i4tile_dword(q, cols / 256, row, c0);
    if (!inverse) {
        const uint8_t *r = src + (size_t)row * (cols / 2);
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) w |= g53_i4_get(r, c0 + 8 * i) << (4 * i);
        ((uint32_t *)dst)[q] = w;
    } else {
        /* column c0 + 8 i has the parity of c0: the eight levels are all low or all high nibbles of
         * eight bytes four apart, which this thread alone writes half of; the other half belongs to
         * the run of the neighbouring accumulator (c0 ^ 1), so the byte is assembled from both */
        const uint32_t w = ((const uint32_t *)src)[q];
        const long q2 = q ^ 16;                      /* run p ^ 4: accumulator c0 ^ 1, same group */
        const uint32_t w2 = ((const uint32_t *)src)[q2];
        if (c0 & 1) return;                          /* the even-column thread writes both nibbles */
        uint8_t *r = dst + (size_t)row * (cols / 2);
#pragma unroll
        for (int i = 0; i < 8; i++)
            r[(c0 + 8 * i) >> 1] = (uint8_t)(((w >> (4 * i)) & 15u) | (((w2 >> (4 * i)) & 15u) << 4));
    }
}

} /* namespace */

static int g53_i4tile_shape(int rows, int cols)
{
    if (rows <= 0 || cols <= 0 || rows % 8 || cols % 256)
        return g53h_fail("g53h_tile_i4: a %d x %d matrix cannot be int4-tiled (rows a multiple of 8, columns of 256)",
                         rows, cols);
    return 0;
}

int g53h_tile_i4_on(uint8_t *dst_d, const uint8_t *src_d, int rows, int cols, int inverse, hipStream_t s)
{
    if (g53h_ready() || g53_i4tile_shape(rows, cols)) return -1;
    if (dst_d == src_d) return g53h_fail("g53h_tile_i4: in-place conversion is not supported");
    const long ndw = (long)rows * cols / 8;
    hipLaunchKernelGGL(k_tile_i4, dim3((unsigned)((ndw + 255) / 256)), dim3(256), 0, s, dst_d, src_d, cols, ndw,
                       inverse);
    G53_LAUNCHED("k_tile_i4");
    return 0;
}

extern "C" int g53h_tile_i4(uint8_t *dst_d, const uint8_t *src_d, int rows, int cols, int inverse)
{
    if (g53h_ready()) return -1;
    return g53h_tile_i4_on(dst_d, src_d, rows, cols, inverse, g53h_stream());
}

extern "C" int g53h_tile_i4_host(uint8_t *dst, const uint8_t *src, int rows, int cols, int inverse)
{
    if (rows <= 0 || cols <= 0 || rows % 8 || cols % 256 || dst == src) return -1;
    const long ndw = (long)rows * cols / 8;
    if (inverse) memset(dst, 0, (size_t)rows * cols / 2);
    for (long q = 0; q < ndw; q++) {
        int row, c0;
        g53_i4tile_dword(q, cols / 256, row, c0);
        uint8_t *r = (uint8_t *)(inverse ? dst : src) + (size_t)row * (cols / 2);
        uint32_t *t = (uint32_t *)(inverse ? src : dst) + q;
        if (!inverse) {
            uint32_t w = 0;
            for (int i = 0; i < 8; i++) w |= g53_i4_get(r, c0 + 8 * i) << (4 * i);
            *t = w;
        } else {
            for (int i = 0; i < 8; i++) {
                const int c = c0 + 8 * i;
                r[c >> 1] |= (uint8_t)(((*t >> (4 * i)) & 15u) << (4 * (c & 1)));
            }
        }
    }
    return 0;
}

/* ------------------------------------------------ int4, MFMA-tiled (G53H_MAT_I4 | MTILED) ---- */
namespace {

/* 8-byte piece q of the int4 MFMA-tiled matrix: unit u = q / 64 (row octet u / nb, 128-column
 * block u % nb), lane slot (q % 64) / 2 = 8 g + m, half q % 2: row 8 (u / nb) + m, columns
 * 128 (u % nb) + 64 (g & 1) + 16 (g >> 1) + 32 half .. + 15, i.e. 8 bytes of the row-major row. */
__host__ __device__ inline void g53_i4m_piece(long q, int nb, int &row, int &col0)
{
    const long u = q >> 6;
    const int ls = (int)(q & 63) >> 1, hf = (int)(q & 1), g = ls >> 3, m = ls & 7;
    row = (int)(u / nb) * 8 + m;
    col0 = (int)(u % nb) * 128 + 64 * (g & 1) + 16 * (g >> 1) + 32 * hf;
}

/* Step q of the tiled steps: unit q / 16, half (q / 8) % 2, row q % 8 of the octet. */
__host__ __device__ inline void g53_i4m_step(long q, int nb, int &row, int &grp)
{
    const long u = q >> 4;
    row = (int)(u / nb) * 8 + (int)(q & 7);
    grp = (int)(u % nb) * 2 + (int)((q >> 3) & 1);
}

__global__ void __launch_bounds__(256) k_mtile_i4(uint8_t *__restrict__ dw, float *__restrict__ ds,
                                                  const uint8_t *__restrict__ sw, const float *__restrict__ ss,
                                                  int cols, long npc, long nst, int inverse)
{
    const long q = (long)blockIdx.x * 256 + threadIdx.x;
    const int nb = cols / 128;
    if (q < npc) {
        int row, c0;
        g53_i4m_piece(q, nb, row, c0);
        uint2 *t = (uint2 *)((inverse ? sw : dw) + 8 * q);
        uint2 *r = (uint2 *)((inverse ? dw : sw) + (size_t)row * (cols / 2) + c0 / 2);
        if (inverse) *r = *t;
        else *t = *r;
    }
    if (q < nst) {
        int row, grp;
        g53_i4m_step(q, nb, row, grp);
        if (inverse) ds[(size_t)row * (cols / 64) + grp] = ss[q];
        else ds[q] = ss[(size_t)row * (cols / 64) + grp];
    }
}

}

int g53h_mtile_i4_on(uint8_t *dw, float *ds, const uint8_t *sw, const float *ss, int rows, int cols, int inverse,
                     hipStream_t s)
{
    if (g53h_ready()) return -1;
    if (rows <= 0 || cols <= 0 || rows % 8 || cols % 128)
        return g53h_fail("g53h_mtile_i4: a %d x %d matrix cannot be MFMA-tiled (rows a multiple of 8, columns of 128)",
                         rows, cols);
    if (dw == sw || (const void *)ds == (const void *)ss)
        return g53h_fail("g53h_mtile_i4: in-place conversion is not supported");
    const long npc = (long)rows * cols / 16, nst = (long)rows * (cols / 64);
    hipLaunchKernelGGL(k_mtile_i4, dim3((unsigned)((npc + 255) / 256)), dim3(256), 0, s, dw, ds, sw, ss, cols, npc,
                       nst, inverse);
    G53_LAUNCHED("k_mtile_i4");
    return 0;
}

extern "C" int g53h_mtile_i4(uint8_t *dst_w, float *dst_s, const uint8_t *src_w, const float *src_s, int rows,
                             int cols, int inverse)
{
    if (g53h_ready()) return -1;
    return g53h_mtile_i4_on(dst_w, dst_s, src_w, src_s, rows, cols, inverse, g53h_stream());
}

extern "C" int g53h_mtile_i4_host(uint8_t *dst_w, float *dst_s, const uint8_t *src_w, const float *src_s, int rows,
                                  int cols, int inverse)
{
    if (rows <= 0 || cols <= 0 || rows % 8 || cols % 128 || dst_w == src_w) return -1;
    const int nb = cols / 128;
    const long npc = (long)rows * cols / 16, nst = (long)rows * (cols / 64);
    for (long q = 0; q < npc; q++) {
        int row, c0;
        g53_i4m_piece(q, nb, row, c0);
        uint8_t *r = (uint8_t *)(inverse ? dst_w : src_w) + (size_t)row * (cols / 2) + c0 / 2;
        uint8_t *t = (uint8_t *)(inverse ? src_w : dst_w) + 8 * q;
        if (inverse) memcpy(r, t, 8);
        else memcpy(t, r, 8);
    }
    if (dst_s && src_s)
        for (long q = 0; q < nst; q++) {
            int row, grp;
            g53_i4m_step(q, nb, row, grp);
            if (inverse) dst_s[(size_t)row * (cols / 64) + grp] = src_s[q];
            else dst_s[q] = src_s[(size_t)row * (cols / 64) + grp];
        }
    return 0;
}

int g53h_mtile_f8_on(uint8_t *dst_d, const uint8_t *src_d, int rows, int cols, int inverse, hipStream_t s)
{
    if (g53h_ready() || g53_tile_shape(rows, cols)) return -1;
    if (dst_d == src_d) return g53h_fail("g53h_mtile_f8: in-place conversion is not supported");
    const long npc = (long)rows * cols / 16;
    hipLaunchKernelGGL(k_mtile_f8, dim3((unsigned)((npc + 255) / 256)), dim3(256), 0, s, dst_d, src_d, cols, npc,
                       inverse);
    G53_LAUNCHED("k_mtile_f8");
    return 0;
}

extern "C" int g53h_mtile_f8(uint8_t *dst_d, const uint8_t *src_d, int rows, int cols, int inverse)
{
    if (g53h_ready()) return -1;
    return g53h_mtile_f8_on(dst_d, src_d, rows, cols, inverse, g53h_stream());
}

extern "C" int g53h_mtile_f8_host(uint8_t *dst, const uint8_t *src, int rows, int cols, int inverse)
{
    if (rows <= 0 || cols <= 0 || rows % 8 || cols % 128 || dst == src) return -1;
    const long npc = (long)rows * cols / 16;
    for (long q = 0; q < npc; q++) {
        int row, c0;
        g53_mtile_piece(q, cols / 128, row, c0);
        for (int j = 0; j < 16; j++) {
            if (inverse) dst[(size_t)row * cols + c0 + j] = src[16 * q + j];
            else dst[16 * q + j] = src[(size_t)row * cols + c0 + j];
        }
    }
    return 0;
}
