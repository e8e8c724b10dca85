/* g53h_rowdot.h - the reference's per-block sums, shared by the kernels that compute one
 * column block (FP8) or group (int4) of a row at a time. */
#ifndef G53H_ROWDOT_H
#define G53H_ROWDOT_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "g53h_core.h"

/* E4M3FN code -> float by the gfx950 conversion instruction (exact; 0x7f / 0xff give NaN, as
 * g53_e4m3_to_f32 and the reference's table). */
__device__ __forceinline__ static float g53_e4m3_hw(uint8_t b) { return __builtin_amdgcn_cvt_f32_fp8((int)b, 0); }

/* The reference's per-block arithmetic (src/core/glm53f_ops.c:195-227): eight fp32 lanes of
 * fused products stepping by 8 columns, reduced in double by a fixed tree, the block tail
 * added in double, the block sum scaled in double and accumulated over blocks in order. */
__device__ __forceinline__ static double g53_block_dot(const uint8_t *row, const float *x, int j0, int j1)
{
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int j = j0;
    for (; j + 8 <= j1; j += 8)
        for (int l = 0; l < 8; l++) a[l] = __builtin_fmaf(g53_e4m3_hw(row[j + l]), x[j + l], a[l]);
    double bsum = (((double)a[0] + a[4]) + ((double)a[2] + a[6]))
                + (((double)a[1] + a[5]) + ((double)a[3] + a[7]));
    for (; j < j1; j++) bsum += (double)g53_e4m3_hw(row[j]) * (double)x[j];
    return bsum;
}

/* The int4 format's group sum (src/core/glm53f_ops.c:247-287): the same eight fp32 lanes over
 * levels (nibble - 8, the even column in the low nibble), the double tree, the tail in double. */
__device__ __forceinline__ static double g53_group_dot_i4(const uint8_t *row, const float *x, int j0, int j1)
{
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int j = j0;
    for (; j + 8 <= j1; j += 8)
        for (int l = 0; l < 8; l++) {
            const uint8_t b = row[(j + l) >> 1];
            const int lv = (int)(((j + l) & 1) ? (b >> 4) : (b & 15)) - 8;
            a[l] = __builtin_fmaf((float)lv, x[j + l], a[l]);
        }
    double bsum = (((double)a[0] + a[4]) + ((double)a[2] + a[6]))
                + (((double)a[1] + a[5]) + ((double)a[3] + a[7]));
    for (; j < j1; j++) {
        const uint8_t b = row[j >> 1];
        const int lv = (int)((j & 1) ? (b >> 4) : (b & 15)) - 8;
        bsum += (double)lv * (double)x[j];
    }
    return bsum;
}

#endif /* G53H_ROWDOT_H */
