/* g53h_synth_host.c - host twins of the seeded synthetic generator (same bits as the
 * device kernel k_synth_f8; see g53h_core.h for the method). */
#include <stddef.h>
#include <stdint.h>

#include "g53h.h"
#include "g53h_core.h"

void g53h_synth_f8_host(uint8_t *w, float *s, int rows, int cols, int br, int bc,
                        uint64_t seed, uint64_t stream, float sigma)
{
    const uint64_t key = g53_key(seed, stream);
    const int srows = (rows + br - 1) / br, scols = (cols + bc - 1) / bc;
    int blk;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1)
#endif
    for (blk = 0; blk < srows * scols; blk++) {
        const int bi = blk / scols, bj = blk % scols;
        const int r0 = bi * br, c0 = bj * bc;
        const int nr = br < rows - r0 ? br : rows - r0, nc = bc < cols - c0 ? bc : cols - c0;
        float amax = 0.0f;
        for (int r = r0; r < r0 + nr; r++)
            for (int c = c0; c < c0 + nc; c++) {
                const float v = g53_normal(key, (uint64_t)r * cols + c, sigma);
                const float a = v < 0 ? -v : v;
                if (a > amax) amax = a;
            }
        const float scale = g53_block_scale(amax);
        for (int r = r0; r < r0 + nr; r++)
            for (int c = c0; c < c0 + nc; c++)
                w[(size_t)r * cols + c] = g53_quant(g53_normal(key, (uint64_t)r * cols + c, sigma), scale);
        s[(size_t)bi * scols + bj] = 1.0f / scale;
    }
}

void g53h_synth_normal_host(float *out, size_t n, uint64_t seed, uint64_t stream, float sigma,
                            int bf16)
{
    const uint64_t key = g53_key(seed, stream);
    long i;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (n > 65536)
#endif
    for (i = 0; i < (long)n; i++) {
        float v = g53_normal(key, (uint64_t)i, sigma);
        if (bf16) v = g53_bitsf((uint32_t)g53_f32_to_bf16(v) << 16);
        out[i] = v;
    }
}

void g53h_synth_uniform_host(float *out, size_t n, uint64_t seed, uint64_t stream, float a)
{
    const uint64_t key = g53_key(seed, stream);
    for (size_t i = 0; i < n; i++) out[i] = g53_uniform_sym(key, (uint64_t)i, a);
}

void g53h_expf_host(float *y, const float *x, size_t n)
{
    long i;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (n > 65536)
#endif
    for (i = 0; i < (long)n; i++) y[i] = g53_expf(x[i]);
}

void g53h_quant_host(uint8_t *q, const float *x, size_t n, float scale)
{
    for (size_t i = 0; i < n; i++) q[i] = g53_quant(x[i], scale);
}
