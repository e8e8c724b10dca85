/* g53h_core.h - arithmetic shared by the gfx950 kernels and the host side of the library.
 *
 * Everything here is written once and compiled twice (HIP device code and plain C host
 * code) so that the two produce the same bits:
 *
 *   g53_expf / g53_sigmoidf   the single-precision exponential the reference's sigmoid
 *                             calls (src/core/glm53f_ops.c:46 uses libm expf). glibc 2.35 on
 *                             x86-64 with FMA implements expf by the table-driven method of
 *                             Szabolcs Nagy (ARM optimized-routines, math/expf.c): x/ln2 is
 *                             scaled by N = 32, rounded with the 1.5*2^52 shift, the
 *                             fractional part r goes through a cubic for 2^(r/N) and the
 *                             integer part indexes a 32-entry table of 2^(i/N). This is our
 *                             own restatement of that published method; the table is
 *                             computed from its definition (2^(i/32) rounded to double, minus
 *                             i << 47) and the cubic coefficients are the published minimax
 *                             ones. With r formed by one fused multiply-add, as the FMA
 *                             build of glibc forms it, the result equals glibc's expf for
 *                             every one of the 2^32 float inputs (checked exhaustively by the
 *                             tests on the host, and against the GPU).
 *   g53_e4m3_to_f32           E4M3FN code -> float (reference src/core/glm53f_ops.c:48-72).
 *   g53_f32_to_e4m3           float -> E4M3FN, round to nearest even, saturating at 448.
 *   synthetic generator       counter-based seeded inputs (see below).
 */
#ifndef G53H_CORE_H
#define G53H_CORE_H

#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define G53_HD __host__ __device__ static inline
#define G53_FMA(a, b, c) __builtin_fma((a), (b), (c))
#else
#include <math.h>
#include <string.h>
#define G53_HD static inline
#define G53_FMA(a, b, c) fma((a), (b), (c))
#endif

G53_HD uint32_t g53_fbits(float f) { union { float f; uint32_t u; } v; v.f = f; return v.u; }
G53_HD float g53_bitsf(uint32_t u) { union { float f; uint32_t u; } v; v.u = u; return v.f; }
G53_HD uint64_t g53_dbits(double d) { union { double d; uint64_t u; } v; v.d = d; return v.u; }
G53_HD double g53_bitsd(uint64_t u) { union { double d; uint64_t u; } v; v.u = u; return v.d; }

/* 2^(i/32) as a double with i << 47 removed from its bit pattern, i = 0..31. */
#define G53_EXP2_TAB { \
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull }

#if defined(__HIPCC__)
__constant__ static const uint64_t g53_exp2_tab_dev[32] = G53_EXP2_TAB;
#endif
static const uint64_t g53_exp2_tab_host[32] = G53_EXP2_TAB;

/* The exponential with the table passed in (kernels keep a copy of it in LDS, so that the
 * per-lane lookup is an LDS read rather than a global load). */
G53_HD float g53_expf_tab(float x, const uint64_t *tab)
{
    const uint32_t ix = g53_fbits(x);
    const uint32_t abstop = (ix >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                       /* |x| >= 88, inf or nan */
        if (ix == 0xff800000u) return 0.0f;      /* -inf */
        if (abstop >= 0x7f8) return x + x;       /* +inf or nan */
        if (x > 0x1.62e42ep6f) return g53_bitsf(0x7f800000u);   /* overflow */
        if (x < -0x1.9fe368p6f) return 0.0f;     /* underflow */
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    const double z = inv_ln2_n * xd;
    double kd = z + shift;
    const uint64_t ki = g53_dbits(kd);
    kd -= shift;
    const double r = G53_FMA(inv_ln2_n, xd, -kd);
    uint64_t t = tab[ki & 31];
    t += ki << 47;
    const double s = g53_bitsd(t);
    const double p = G53_FMA(c0, r, c1);
    const double r2 = r * r;
    double y = G53_FMA(c2, r, 1.0);
    y = G53_FMA(p, r2, y);
    y = y * s;
    return (float)y;
}

G53_HD float g53_expf(float x)
{
#if defined(__HIP_DEVICE_COMPILE__)
    return g53_expf_tab(x, g53_exp2_tab_dev);
#else
    return g53_expf_tab(x, g53_exp2_tab_host);
#endif
}

/* 1 / (1 + e^-x) in float, operation for operation as the reference's sigmoidf_. */
G53_HD float g53_sigmoidf_tab(float x, const uint64_t *tab)
{
    const float e = g53_expf_tab(-x, tab);
    const float d = 1.0f + e;
    return 1.0f / d;
}

/* SwiGLU with the clamp: the gate only from above, the up projection both ways
 * (reference src/core/glm53f_ops.c:486-494). */
G53_HD float g53_swiglu1_tab(float g, float u, float limit, const uint64_t *tab)
{
    const float gi = g > limit ? limit : g;
    const float ui = u > limit ? limit : (u < -limit ? -limit : u);
    const float sg = gi * g53_sigmoidf_tab(gi, tab);
    return sg * ui;
}

#if defined(__HIP_DEVICE_COMPILE__)
#define G53_EXP_TAB g53_exp2_tab_dev
#else
#define G53_EXP_TAB g53_exp2_tab_host
#endif
G53_HD float g53_sigmoidf(float x) { return g53_sigmoidf_tab(x, G53_EXP_TAB); }
G53_HD float g53_swiglu1(float g, float u, float limit) { return g53_swiglu1_tab(g, u, limit, G53_EXP_TAB); }

/* E4M3FN: sign, 4-bit exponent (bias 7), 3-bit mantissa, no infinities, 0x7f/0xff NaN. */
G53_HD float g53_e4m3_to_f32(uint8_t b)
{
    const uint32_t s = (uint32_t)(b >> 7) << 31, e = (b >> 3) & 15u, m = b & 7u;
    if (e == 15 && m == 7) return g53_bitsf(s | 0x7fc00000u);
    if (e == 0) {                                /* m/8 * 2^-6, exact in float */
        if (m == 0) return g53_bitsf(s);
        uint32_t mm = m, ee = 127 - 9;           /* value = m * 2^-9 */
        while (!(mm & 8)) { mm <<= 1; ee--; }
        return g53_bitsf(s | (ee + 3) << 23 | (mm & 7u) << 20);
    }
    return g53_bitsf(s | (e + 120u) << 23 | m << 20);
}

/* float -> E4M3FN, round to nearest, ties to even; |f| above 448 saturates to 448, NaN maps
 * to 0x7f with the sign kept. */
G53_HD uint8_t g53_f32_to_e4m3(float f)
{
    const uint32_t u = g53_fbits(f);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint8_t)(sign | 0x7f);
    if (a >= 0x43e00000u) return (uint8_t)(sign | 0x7e);          /* >= 448 */
    const uint32_t E = a >> 23;
    if (E < 121) {                               /* below 2^-6: multiples of 2^-9 */
        if (E == 0) return (uint8_t)sign;        /* float subnormal: rounds to zero */
        const uint32_t M = (a & 0x7fffffu) | 0x800000u;
        const uint32_t sh = 141 - E;             /* >= 21 */
        if (sh > 24) return (uint8_t)sign;       /* below half of 2^-9 */
        uint32_t q = M >> sh;
        const uint32_t rem = M & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint8_t)(sign | q);              /* q == 8 is the smallest normal, 0x08 */
    }
    uint32_t q = (a & 0x7fffffu) >> 20;
    const uint32_t rem = a & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) q++;
    uint32_t code = ((E - 120u) << 3) + q;
    if (code > 0x7eu) code = 0x7eu;
    return (uint8_t)(sign | code);
}

/* float -> bf16 bits, round to nearest even (finite inputs). */
G53_HD uint16_t g53_f32_to_bf16(float f)
{
    const uint32_t u = g53_fbits(f);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

/* ---------------------------------------------------------- synthetic generator ----
 * Counter-based, so any element can be produced alone and the device and the host produce
 * the same bits. A 64-bit key comes from (seed, stream); element n of a stream draws six
 * splitmix64 outputs (Steele, Lea and Flood 2014: golden-gamma increment then the
 * variant-13 finalizer), each giving two 24-bit uniforms. The sum of the twelve, minus
 * 6 * 2^24, is an Irwin-Hall approximation of N(0,1) in units of 2^-24: mean 0, variance 1,
 * integer arithmetic only, so it is exact on both sides. Scaling to sigma is one float
 * rounding of (float)S * (sigma * 2^-24). */
G53_HD uint64_t g53_fin64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

G53_HD uint64_t g53_key(uint64_t seed, uint64_t stream)
{
    return g53_fin64(seed * 0x9e3779b97f4a7c15ull + g53_fin64(stream + 0x632be59bd9b4e019ull));
}

G53_HD uint64_t g53_rand64(uint64_t key, uint64_t n)
{
    return g53_fin64(key + (n + 1) * 0x9e3779b97f4a7c15ull);
}

/* Irwin-Hall(12) - 6 in units of 2^-24. */
G53_HD int32_t g53_normal_units(uint64_t key, uint64_t i)
{
    int32_t s = 0;
    for (int k = 0; k < 6; k++) {
        const uint64_t h = g53_rand64(key, i * 6 + (uint64_t)k);
        s += (int32_t)(h & 0xffffffu) + (int32_t)((h >> 32) & 0xffffffu);
    }
    return s - 100663296;                        /* 6 * 2^24 */
}

/* N(0, sigma^2) approximation; sigma * 2^-24 must be a normal float. */
G53_HD float g53_normal(uint64_t key, uint64_t i, float sigma)
{
    const float unit = sigma * 0x1p-24f;
    return (float)g53_normal_units(key, i) * unit;
}

/* U(-a, a) on a 2^24 grid. */
G53_HD float g53_uniform_sym(uint64_t key, uint64_t i, float a)
{
    const int32_t v = (int32_t)(g53_rand64(key, i) & 0xffffffu) - 0x800000;
    return (float)v * (a * 0x1p-23f);
}

/* One FP8 block quantised by the absmax rule of the reference's fixture generator
 * (tools/make_glm_tiny.py:50-62): scale = 448 / max|w| (1 if the block is zero), codes =
 * E4M3(clamp(w * scale, +-448)), stored scale = 1 / scale. */
G53_HD float g53_block_scale(float amax) { return amax > 0.0f ? 448.0f / amax : 1.0f; }
G53_HD uint8_t g53_quant(float v, float scale)
{
    float t = v * scale;
    t = t > 448.0f ? 448.0f : (t < -448.0f ? -448.0f : t);
    return g53_f32_to_e4m3(t);
}

#endif /* G53H_CORE_H */
