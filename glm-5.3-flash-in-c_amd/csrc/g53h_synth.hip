/* g53h_synth.hip - seeded synthetic FP8 weights on the device, and the check kernels
 * (expf restatement, E4M3 conversion) that pin the device arithmetic to the host's. */
#include <hip/hip_runtime.h>

#include "g53h.h"
#include "g53h_core.h"
#include "g53h_runtime.h"

/* One workgroup per (br x bc) block: pass 1 finds max|w| over the block, pass 2 draws the
 * same elements again and writes the codes; one thread writes the block scale. */
__global__ void __launch_bounds__(256) k_synth_f8(uint8_t *__restrict__ w, float *__restrict__ s,
                                                  int rows, int cols, int br, int bc, int scols,
                                                  uint64_t key, float sigma)
{
    const int bi = blockIdx.y, bj = blockIdx.x;
    const int r0 = bi * br, c0 = bj * bc;
    const int nr = min(br, rows - r0), nc = min(bc, cols - c0);
    const int n = nr * nc;
    float amax = 0.0f;
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        const int r = r0 + e / nc, c = c0 + e % nc;
        const float v = g53_normal(key, (uint64_t)r * cols + c, sigma);
        amax = fmaxf(amax, fabsf(v));
    }
    for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    __shared__ float red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float scale = g53_block_scale(amax);
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        const int r = r0 + e / nc, c = c0 + e % nc;
        const float v = g53_normal(key, (uint64_t)r * cols + c, sigma);
        w[(size_t)r * cols + c] = g53_quant(v, scale);
    }
    if (threadIdx.x == 0) s[(size_t)bi * scols + bj] = 1.0f / scale;
}

extern "C" int g53h_synth_f8(uint8_t *w, float *s, int rows, int cols, int br, int bc,
                             uint64_t seed, uint64_t stream, float sigma)
{
    if (g53h_ready()) return -1;
    if (rows <= 0 || cols <= 0 || br <= 0 || bc <= 0) return g53h_fail("g53h_synth_f8: bad shape");
    const int srows = (rows + br - 1) / br, scols = (cols + bc - 1) / bc;
    dim3 grid(scols, srows);
    hipLaunchKernelGGL(k_synth_f8, grid, dim3(256), 0, g53h_stream(), w, s, rows, cols, br, bc,
                       scols, g53_key(seed, stream), sigma);
    G53_LAUNCHED("k_synth_f8");
    return 0;
}

__global__ void k_expf(float *__restrict__ y, const float *__restrict__ x, size_t n)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = g53_expf(x[i]);
}

__global__ void k_expf_range(float *__restrict__ y, uint32_t base, size_t n)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = g53_expf(g53_bitsf(base + (uint32_t)i));
}

extern "C" int g53h_expf(float *y, const float *x, size_t n)
{
    if (g53h_ready()) return -1;
    if (!n) return 0;
    hipLaunchKernelGGL(k_expf, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, g53h_stream(), y, x, n);
    G53_LAUNCHED("k_expf");
    return 0;
}

extern "C" int g53h_expf_range(float *y, uint32_t base, size_t n)
{
    if (g53h_ready()) return -1;
    if (!n) return 0;
    if (n > (1ull << 32)) return g53h_fail("g53h_expf_range: n above 2^32");
    hipLaunchKernelGGL(k_expf_range, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, g53h_stream(),
                       y, base, n);
    G53_LAUNCHED("k_expf_range");
    return 0;
}

typedef float g53_f2 __attribute__((ext_vector_type(2)));

/* Four codes per thread through v_cvt_pk_f32_fp8, the conversion the GEMV kernels use. */
__global__ void k_e4m3_decode(float *__restrict__ out, const uint8_t *__restrict__ codes, size_t n)
{
    const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i >= n) return;
    uint32_t v = 0;
    for (int k = 0; k < 4 && i + k < n; k++) v |= (uint32_t)codes[i + k] << (8 * k);
    const g53_f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)v, false);
    const g53_f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)v, true);
    const float f[4] = {lo[0], lo[1], hi[0], hi[1]};
    for (int k = 0; k < 4 && i + k < n; k++) out[i + k] = f[k];
}

extern "C" int g53h_e4m3_decode(float *out, const uint8_t *codes, size_t n)
{
    if (g53h_ready()) return -1;
    if (!n) return 0;
    const size_t th = (n + 3) / 4;
    hipLaunchKernelGGL(k_e4m3_decode, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, g53h_stream(),
                       out, codes, n);
    G53_LAUNCHED("k_e4m3_decode");
    return 0;
}
