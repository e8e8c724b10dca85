/* g53_oracle.c - CPU restatement of the reference's routed-expert MoE path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product links or calls this file: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the checker. Each
 * function restates the reference operation for operation (josesilva05/glm-5.3-flash-in-c,
 * file:line cited per function) in plain scalar C; it is compiled with -ffp-contract=off so
 * that every multiply and add the reference keeps apart stays apart, and fmaf/fma are called
 * exactly where the reference fuses.
 *
 * How each function is pinned (tests/test_oracle.py):
 *   or_e4m3f        closed form over all 256 codes, and the reference's table via oracle/_ref
 *   or_mm_f8        the reference's own known-answer inputs (tests/unit/test_fp8.c:38-54,
 *                   150-157) against golden outputs of the compiled reference, bit for bit;
 *                   and a dequantise-then-fp64 bound
 *   or_swiglu       closed form
 *   or_router       brute force (fp64 dot + sort) on small inputs; golden vectors
 *   or_route_topn   brute force on small inputs, NaN rules by hand-made cases
 *   or_moe          golden vectors of the compiled reference (configs 1-2 shapes and the
 *                   reference's glm_tiny fixture weights), bit for bit
 *   or_i4_from_f8   (tests/test_oracle_i4.py) the reference's quantiser known-answer case
 *                   (tests/unit/test_fp8.c:161) by digest of the compiled reference's output,
 *                   its half-a-step property, hand-made groups, unaligned scale blocks (golden)
 *   or_mm_i4        the reference's int4 known-answer cases (tests/unit/test_fp8.c:158-160),
 *                   golden, bit for bit; a dequantise-then-fp64 bound; a ragged group by hand
 *   or_moe_i4       golden outputs of the compiled reference with int4 routed experts
 *                   (configs 1-2), and the weighted sum of separately run int4 experts
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* E4M3FN decode (reference src/core/glm53f_ops.c:50-66): e == 0 subnormal m/8*2^-6,
 * otherwise (1 + m/8) * 2^(e-7); exponent 15 with mantissa 7 is NaN. */
float or_e4m3f(uint8_t b)
{
    const int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
    double v;
    if (e == 15 && m == 7) v = NAN;
    else if (e == 0) v = ldexp((double)m / 8.0, -6);
    else v = ldexp(1.0 + (double)m / 8.0, e - 7);
    return (float)(s ? -v : v);
}

/* 1/(1+expf(-x)) (reference src/core/glm53f_ops.c:46). */
static float or_sigmoidf(float x) { return 1.0f / (1.0f + expf(-x)); }

/* FP8 block-scaled matvec (reference src/core/glm53f_ops.c:185-228; the scalar form of
 * tests/unit/test_fp8.c:16-36). y[t][rows] for x[t][cols]; the batched form
 * (src/core/glm53f_ops.c:378-427) is the same sum per token. */
void or_mm_f8(float *y, const float *x, int T, const uint8_t *W, const float *S, int rows,
              int cols, int br, int bc)
{
    const int scols = (cols + bc - 1) / bc;
    long i;
#pragma omp parallel for schedule(static)
    for (i = 0; i < (long)T * rows; i++) {
        const int t = (int)(i / rows), o = (int)(i % rows);
        const float *xt = x + (size_t)t * cols;
        const uint8_t *row = W + (size_t)o * cols;
        const float *srow = S + (size_t)(o / br) * scols;
        double acc = 0.0;
        for (int b = 0, j0 = 0; j0 < cols; b++, j0 += bc) {
            const int j1 = (j0 + bc < cols) ? j0 + bc : cols;
            int j = j0;
            float a[8] = {0};
            for (; j + 8 <= j1; j += 8)
                for (int l = 0; l < 8; l++) a[l] = fmaf(or_e4m3f(row[j + l]), xt[j + l], a[l]);
            double bsum = (((double)a[0] + a[4]) + ((double)a[2] + a[6]))
                        + (((double)a[1] + a[5]) + ((double)a[3] + a[7]));
            for (; j < j1; j++) bsum += (double)or_e4m3f(row[j]) * (double)xt[j];
            acc += bsum * (double)srow[b];
        }
        y[(size_t)t * rows + o] = (float)acc;
    }
}

/* SwiGLU with clamp (reference src/core/glm53f_ops.c:486-494). */
void or_swiglu(float *y, const float *gu, int n, float limit)
{
    const float *g = gu, *u = gu + n;
    for (int i = 0; i < n; i++) {
        float gi = g[i] > limit ? limit : g[i];
        float ui = u[i] > limit ? limit : (u[i] < -limit ? -limit : u[i]);
        y[i] = (gi * or_sigmoidf(gi)) * ui;
    }
}

/* Router (reference src/core/glm53f_ops.c:945-976). Returns -1 where the reference aborts
 * (no selectable candidate), else 0. */
int or_router(int *idx, float *w, const float *x, const float *gate, const float *bias, int NE,
              int E, int K, int norm_topk, float routed_scale)
{
    float *score = (float *)malloc((size_t)NE * sizeof(float));
    float *choice = (float *)malloc((size_t)NE * sizeof(float));
    int ret = 0;
    for (int e = 0; e < NE; e++) {
        const float *row = gate + (size_t)e * E;
        double acc = 0.0;
        for (int i = 0; i < E; i++) acc += (double)row[i] * (double)x[i];
        score[e] = or_sigmoidf((float)acc);
        choice[e] = score[e] + bias[e];
    }
    for (int j = 0; j < K; j++) {
        int best = -1;
        float bv = -INFINITY;
        for (int ee = 0; ee < NE; ee++)
            if (choice[ee] > bv) { bv = choice[ee]; best = ee; }
        if (best < 0) { ret = -1; best = 0; }
        idx[j] = best;
        w[j] = score[best];
        choice[best] = -INFINITY;
    }
    if (norm_topk) {
        double s = 0.0;
        for (int j = 0; j < K; j++) s += (double)w[j];
        for (int j = 0; j < K; j++) w[j] = (float)((double)w[j] / (s + 1e-20));
    }
    for (int j = 0; j < K; j++) w[j] *= routed_scale;
    free(score);
    free(choice);
    return ret;
}

/* Next-layer prediction (reference src/core/glm53f_ops.c:1021-1042). */
void or_route_topn(int *idx, int n, const float *x, const float *gate, const float *bias, int NE,
                   int E)
{
    float *choice = (float *)malloc((size_t)NE * sizeof(float));
    for (int e = 0; e < NE; e++) {
        const float *row = gate + (size_t)e * E;
        double acc = 0.0;
        for (int i = 0; i < E; i++) acc += (double)row[i] * (double)x[i];
        choice[e] = or_sigmoidf((float)acc) + bias[e];
    }
    for (int j = 0; j < n; j++) {
        int best = 0;
        for (int ee = 1; ee < NE; ee++) if (choice[ee] > choice[best]) best = ee;
        idx[j] = best;
        choice[best] = -INFINITY;
    }
    free(choice);
}

typedef struct {
    const uint8_t *gw, *uw, *dw;      /* gate [I][E], up [I][E], down [E][I]; gw NULL = dropped */
    const float   *gs, *us, *ds;
} OrExpert;

/* One MoE layer over T tokens (reference src/core/glm53f_ops.c:1144-1342 moe_chunk, as
 * driven by glm53f_moe :1344-1351): route every token, apply each chosen expert (a dropped
 * expert contributes zero, :1261-1270), combine per token in double in slot order (:1329-1337)
 * and add the shared expert in float (:1338-1340) when shared != NULL. idx_out / w_out
 * ([T][K], optional) receive the routing. Returns -1 where the reference aborts. */
int or_moe(float *out, const float *x, int T, int E, int I, int NE, int K, int br, int bc,
           int norm_topk, float routed_scale, float limit, const float *gate, const float *bias,
           const OrExpert *experts, const OrExpert *shared, int *idx_out, float *w_out)
{
    int *ids = (int *)malloc((size_t)K * sizeof(int));
    float *wts = (float *)malloc((size_t)K * sizeof(float));
    float *contrib = (float *)malloc((size_t)K * E * sizeof(float));
    float *gu = (float *)malloc((size_t)2 * I * sizeof(float));
    float *act = (float *)malloc((size_t)I * sizeof(float));
    float *sho = (float *)malloc((size_t)E * sizeof(float));
    int ret = 0;
    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * E;
        if (or_router(ids, wts, xt, gate, bias, NE, E, K, norm_topk, routed_scale)) ret = -1;
        if (idx_out) memcpy(idx_out + (size_t)t * K, ids, (size_t)K * sizeof(int));
        if (w_out) memcpy(w_out + (size_t)t * K, wts, (size_t)K * sizeof(float));
        for (int j = 0; j < K; j++) {
            const OrExpert *ex = &experts[ids[j]];
            float *dst = contrib + (size_t)j * E;
            if (!ex->gw) { memset(dst, 0, (size_t)E * sizeof(float)); continue; }
            or_mm_f8(gu, xt, 1, ex->gw, ex->gs, I, E, br, bc);
            or_mm_f8(gu + I, xt, 1, ex->uw, ex->us, I, E, br, bc);
            or_swiglu(act, gu, I, limit);
            or_mm_f8(dst, act, 1, ex->dw, ex->ds, E, I, br, bc);
        }
        float *ot = out + (size_t)t * E;
        for (int d = 0; d < E; d++) {
            double s = 0.0;
            for (int j = 0; j < K; j++) s += (double)wts[j] * (double)contrib[(size_t)j * E + d];
            ot[d] = (float)s;
        }
        if (shared) {
            or_mm_f8(gu, xt, 1, shared->gw, shared->gs, I, E, br, bc);
            or_mm_f8(gu + I, xt, 1, shared->uw, shared->us, I, E, br, bc);
            or_swiglu(act, gu, I, limit);
            or_mm_f8(sho, act, 1, shared->dw, shared->ds, E, I, br, bc);
            for (int d = 0; d < E; d++) ot[d] += sho[d];
        }
    }
    free(ids); free(wts); free(contrib); free(gu); free(act); free(sho);
    return ret;
}

/* ------------------------------------------------------------------ int4 ---- */
/* FP8 -> int4 re-quantisation (reference src/core/glm53f_ops.c:303-371, glm53f_i4_from_f8):
 * per row and group of 64 columns, vals = the decoded codes (times the block scale when the
 * group straddles scale blocks), amax = max |vals|, step = (aligned ? amax * blockscale : amax)
 * / 7 (floored at 1e-30), level = clamp(rint(val * (aligned ? 7 / amax : 1 / step)), -8, 7),
 * stored as level + 8, two per byte, the even column in the low nibble. q [rows][cols/2],
 * steps [rows][cols/64]. */
#define OR_I4_GROUP 64
void or_i4_from_f8(uint8_t *q, float *steps, const uint8_t *W, const float *S, int rows, int cols, int br,
                   int bc)
{
    const int gs = OR_I4_GROUP, groups = cols / gs, scols = (cols + bc - 1) / bc;
    for (int o = 0; o < rows; o++) {
        const uint8_t *row = W + (size_t)o * cols;
        const float *srow = S + (size_t)(o / br) * scols;
        for (int g = 0; g < groups; g++) {
            const int j0 = g * gs, aligned = bc % gs == 0;
            const float bs = srow[j0 / bc];
            float vals[OR_I4_GROUP], amax = 0.0f;
            for (int j = 0; j < gs; j++) {
                const float w = or_e4m3f(row[j0 + j]) * (aligned ? 1.0f : srow[(j0 + j) / bc]);
                vals[j] = w;
                const float a = w < 0.0f ? -w : w;
                if (a > amax) amax = a;
            }
            float step = (aligned ? amax * bs : amax) / 7.0f;
            if (!(step > 1e-30f)) step = 1e-30f;
            steps[(size_t)o * groups + g] = step;
            const float inv = amax > 0.0f ? 7.0f / amax : 0.0f;
            const float mul = aligned ? inv : (1.0f / step);
            for (int j = 0; j < gs; j += 2) {
                int l0 = (int)lrintf(vals[j] * mul), l1 = (int)lrintf(vals[j + 1] * mul);
                l0 = l0 < -8 ? -8 : (l0 > 7 ? 7 : l0);
                l1 = l1 < -8 ? -8 : (l1 > 7 ? 7 : l1);
                q[(size_t)o * (cols / 2) + ((j0 + j) >> 1)] = (uint8_t)((l0 + 8) | ((l1 + 8) << 4));
            }
        }
    }
}

/* The int4 matrix-vector product (reference src/core/glm53f_ops.c:236-296, matmul_i4): per row
 * and group of gs columns eight fp32 lanes a[l] = fmaf(level, x, a[l]) stepping by 8, the double
 * tree, the tail in double, times the group's step in double, added over the row's groups in
 * order. */
void or_mm_i4(float *y, const float *x, int T, const uint8_t *Q, const float *steps, int rows, int cols, int gs)
{
    const int groups = (cols + gs - 1) / gs;
    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * cols;
        for (int o = 0; o < rows; o++) {
            const uint8_t *row = Q + (size_t)o * (cols / 2);
            double acc = 0.0;
            for (int g = 0; g < groups; g++) {
                const int j0 = g * gs, j1 = j0 + gs < cols ? j0 + gs : cols;
                float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                int j = j0;
                for (; j + 8 <= j1; j += 8)
                    for (int l = 0; l < 8; l++) {
                        const uint8_t b = row[(j + l) >> 1];
                        const int lv = (int)(((j + l) & 1) ? (b >> 4) : (b & 0x0f)) - 8;
                        a[l] = fmaf((float)lv, xt[j + l], a[l]);
                    }
                double bsum = (((double)a[0] + a[4]) + ((double)a[2] + a[6])) + (((double)a[1] + a[5]) + ((double)a[3] + a[7]));
                for (; j < j1; j++) {
                    const uint8_t b = row[j >> 1];
                    const int lv = (int)((j & 1) ? (b >> 4) : (b & 0x0f)) - 8;
                    bsum += (double)lv * (double)xt[j];
                }
                acc += bsum * (double)steps[(size_t)o * groups + g];
            }
            y[(size_t)t * rows + o] = (float)acc;
        }
    }
}

/* or_moe with int4 routed experts (q, steps per matrix; the shared expert stays FP8, as the
 * reference's int4 cache holds only routed experts). */
typedef struct {
    const uint8_t *gq, *uq, *dq;      /* gq NULL = dropped */
    const float   *gs, *us, *ds;      /* steps */
} OrExpertI4;

int or_moe_i4(float *out, const float *x, int T, int E, int I, int NE, int K, int br, int bc, int norm_topk,
              float routed_scale, float limit, const float *gate, const float *bias, const OrExpertI4 *experts,
              const OrExpert *shared, int *idx_out, float *w_out)
{
    int *ids = (int *)malloc((size_t)K * sizeof(int));
    float *wts = (float *)malloc((size_t)K * sizeof(float));
    float *contrib = (float *)malloc((size_t)K * E * sizeof(float));
    float *gu = (float *)malloc((size_t)2 * I * sizeof(float));
    float *act = (float *)malloc((size_t)I * sizeof(float));
    float *sho = (float *)malloc((size_t)E * sizeof(float));
    int ret = 0;
    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * E;
        if (or_router(ids, wts, xt, gate, bias, NE, E, K, norm_topk, routed_scale)) ret = -1;
        if (idx_out) memcpy(idx_out + (size_t)t * K, ids, (size_t)K * sizeof(int));
        if (w_out) memcpy(w_out + (size_t)t * K, wts, (size_t)K * sizeof(float));
        for (int j = 0; j < K; j++) {
            const OrExpertI4 *ex = &experts[ids[j]];
            float *dst = contrib + (size_t)j * E;
            if (!ex->gq) { memset(dst, 0, (size_t)E * sizeof(float)); continue; }
            or_mm_i4(gu, xt, 1, ex->gq, ex->gs, I, E, OR_I4_GROUP);
            or_mm_i4(gu + I, xt, 1, ex->uq, ex->us, I, E, OR_I4_GROUP);
            or_swiglu(act, gu, I, limit);
            or_mm_i4(dst, act, 1, ex->dq, ex->ds, E, I, OR_I4_GROUP);
        }
        float *ot = out + (size_t)t * E;
        for (int d = 0; d < E; d++) {
            double s = 0.0;
            for (int j = 0; j < K; j++) s += (double)wts[j] * (double)contrib[(size_t)j * E + d];
            ot[d] = (float)s;
        }
        if (shared) {
            or_mm_f8(gu, xt, 1, shared->gw, shared->gs, I, E, br, bc);
            or_mm_f8(gu + I, xt, 1, shared->uw, shared->us, I, E, br, bc);
            or_swiglu(act, gu, I, limit);
            or_mm_f8(sho, act, 1, shared->dw, shared->ds, E, I, br, bc);
            for (int d = 0; d < E; d++) ot[d] += sho[d];
        }
    }
    free(ids); free(wts); free(contrib); free(gu); free(act); free(sho);
    return ret;
}

/* Checks of device results against the host C library (glibc expf, as the reference calls it):
 * y[i] is the device's expf of the float with bit pattern base + i. Returns the number of
 * results that differ in any bit (NaN matches NaN); the first mismatch goes to *first. */
long or_expf_mismatches(const float *y, uint32_t base, long n, long *first)
{
    long bad = 0, f = -1;
    long i;
#pragma omp parallel for schedule(static) reduction(+:bad)
    for (i = 0; i < n; i++) {
        union { uint32_t u; float f; } in, a, b;
        in.u = base + (uint32_t)i;
        a.f = expf(in.f);
        b.f = y[i];
        if (a.u != b.u && !(a.f != a.f && b.f != b.f)) {
            bad++;
#pragma omp critical
            if (f < 0 || i < f) f = i;
        }
    }
    if (first) *first = f;
    return bad;
}

void or_expf(float *y, const float *x, long n)
{
    for (long i = 0; i < n; i++) y[i] = expf(x[i]);
}

/* The reference test's generator (tests/unit/test_fp8.c:38-39): rng = rng*1664525 + 1013904223,
 * next() = rng >> 8. Writes n successive next() values and advances *state. */
void or_lcg(uint32_t *state, uint32_t *out, long n)
{
    uint32_t r = *state;
    for (long i = 0; i < n; i++) { r = r * 1664525u + 1013904223u; out[i] = r >> 8; }
    *state = r;
}
