/* glm53f_moe.c - the reference's expert-path entry points, served by the gfx950 kernels.
 *
 * Same signatures and the same observable behaviour as src/core/glm53f_ops.c of the
 * reference: routing, the expert order, the drop path, the hint/prefetch protocol of
 * moe_chunk (src/core/glm53f_ops.c:1144-1342) and the abort-on-error convention. The
 * arithmetic runs on the GPU through g53h.h; this file only moves operands, drives the expert
 * source and keeps weights resident.
 *
 * Host weights (router, bias, shared expert, host expert views) are uploaded to HBM once
 * and found again by their host address in a small open-addressing table; a pointer that is
 * already HBM is used as is. Host expert views (an Glm53fExpertSrc that serves host memory)
 * are copied per call into staging slots instead, since a source may reuse its memory after
 * release().
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "g53h.h"
#include "g53h_core.h"
#include "glm53f.h"
#include "glm53f_cache.h"

long glm53f_expert_drops = 0;
int  glm53f_quiet = 0;
const char *glm53f_i4_dir = NULL;     /* not read: int4 layers are quantised as they land */

#define G53_MOE_CHUNK 64                /* reference chunk (src/core/glm53f_ops.c:988) */

static void g53_die(const char *what)
{
    fprintf(stderr, "glm53f: FATAL, %s: %s\n", what, g53h_error());
    abort();
}

/* ------------------------------------------------------------ resident weights ---- */
/* An entry is found by host address and checked against the host size and 16 words sampled
 * across the bytes, recorded at upload: a caller that frees its weights and reuses the address
 * for others gets them uploaded again instead of the stale copy. Every use compares the first
 * and the last sampled word and one more in rotation (three loads instead of sixteen, since a
 * decode step looks up every layer's weights), so all sixteen are compared every 14 uses. */
#define G53_NSAMP 16
typedef struct { const void *h; size_t n; void *d; int dt; size_t hn; uint64_t samp[G53_NSAMP]; unsigned use; } G53Res;

static uint64_t res_word(const void *h, size_t hn, int k)
{
    uint64_t w = 0;
    if (hn >= 8) memcpy(&w, (const unsigned char *)h + (size_t)k * ((hn - 8) / (G53_NSAMP - 1)), 8);
    return w;
}

static void res_record(G53Res *r, const void *h, size_t hn)
{
    r->hn = hn;
    r->use = 0;
    for (int k = 0; k < G53_NSAMP; k++) r->samp[k] = res_word(h, hn, k);
}

static int res_same(G53Res *r, const void *h, size_t hn)
{
    if (r->hn != hn) return 0;
    const int k = 1 + (int)(r->use++ % (G53_NSAMP - 2));
    return res_word(h, hn, 0) == r->samp[0] && res_word(h, hn, G53_NSAMP - 1) == r->samp[G53_NSAMP - 1] &&
           res_word(h, hn, k) == r->samp[k];
}
static G53Res *g_res = NULL;
static size_t g_res_cap = 0, g_res_n = 0;

static size_t res_hash(const void *p, size_t cap)
{
    uint64_t v = (uint64_t)(uintptr_t)p;
    v ^= v >> 33; v *= 0xff51afd7ed558ccdull; v ^= v >> 33;
    return (size_t)(v & (cap - 1));
}

static G53Res *res_find(const void *h)
{
    if (!g_res_cap) return NULL;
    for (size_t i = res_hash(h, g_res_cap);; i = (i + 1) & (g_res_cap - 1)) {
        if (g_res[i].h == h) return &g_res[i];
        if (!g_res[i].h) return NULL;
    }
}

static G53Res *res_insert(const void *h)
{
    if (2 * (g_res_n + 1) > g_res_cap) {
        const size_t ncap = g_res_cap ? 2 * g_res_cap : 256;
        G53Res *nt = (G53Res *)calloc(ncap, sizeof *nt);
        if (!nt) { fprintf(stderr, "glm53f: FATAL, out of host memory\n"); abort(); }
        for (size_t i = 0; i < g_res_cap; i++) {
            if (!g_res[i].h) continue;
            size_t j = res_hash(g_res[i].h, ncap);
            while (nt[j].h) j = (j + 1) & (ncap - 1);
            nt[j] = g_res[i];
        }
        free(g_res);
        g_res = nt;
        g_res_cap = ncap;
    }
    size_t j = res_hash(h, g_res_cap);
    while (g_res[j].h) j = (j + 1) & (g_res_cap - 1);
    g_res[j].h = h;
    g_res_n++;
    return &g_res[j];
}

/* HBM copy of n host bytes at h (or h itself when it is HBM). */
static const void *resident(const void *h, size_t n)
{
    if (!h) return NULL;
    G53Res *r = res_find(h);                  /* a known host weight: no pointer query */
    if (r && r->n == n && r->dt < 0 && res_same(r, h, n)) return r->d;
    if (g53h_is_device_ptr(h)) return h;
    void *d = g53h_alloc(n);
    if (!d || g53h_h2d(d, h, n)) g53_die("uploading a weight to HBM");
    if (!r) r = res_insert(h);
    else if (g53h_sync() || g53h_free(r->d)) g53_die("replacing a resident weight");
    r->n = n; r->d = d; r->dt = -1;
    res_record(r, h, n);
    return d;
}

/* The router as resident: fp32 rows whose values are all bf16-representable (the released
 * checkpoint stores the router in bf16 and the engine widens it) are kept as bf16, half the
 * bytes for the same exact values. *dt receives 0 (fp32) or 1 (bf16). */
static const void *resident_router(const float *h, size_t n, int *dt)
{
    G53Res *r = res_find(h);
    if (r && r->dt >= 0 && r->n == n * (r->dt ? 2 : 4) && res_same(r, h, n * sizeof(float))) {
        *dt = r->dt;
        return r->d;
    }
    if (g53h_is_device_ptr(h)) { *dt = 0; return h; }
    int bf = 1;
    for (size_t i = 0; i < n && bf; i++) if (g53_fbits(h[i]) & 0xffffu) bf = 0;
    void *d;
    size_t bytes;
    if (bf) {
        uint16_t *tmp = (uint16_t *)malloc(n * 2);
        if (!tmp) { fprintf(stderr, "glm53f: FATAL, out of host memory\n"); abort(); }
        for (size_t i = 0; i < n; i++) tmp[i] = (uint16_t)(g53_fbits(h[i]) >> 16);
        bytes = n * 2;
        d = g53h_alloc(bytes);
        if (!d || g53h_h2d(d, tmp, bytes)) g53_die("uploading the router");
        free(tmp);
    } else {
        bytes = n * 4;
        d = g53h_alloc(bytes);
        if (!d || g53h_h2d(d, h, bytes)) g53_die("uploading the router");
    }
    if (!r) r = res_insert(h);
    else if (g53h_sync() || g53h_free(r->d)) g53_die("replacing a resident router");
    r->n = bytes; r->d = d; r->dt = bf;
    res_record(r, h, n * sizeof(float));
    *dt = bf;
    return d;
}

void glm53f_forget_host_weights(void)
{
    for (size_t i = 0; i < g_res_cap; i++) if (g_res[i].h) g53h_free(g_res[i].d);
    free(g_res);
    g_res = NULL;
    g_res_cap = g_res_n = 0;
}

/* Bytes of a matrix's codes and scales: FP8 [rows][cols] codes and [ceil(rows/br)][scols]
 * scales; int4 (GLM53F_WI4, GLM53F_WI4T with the levels int4-tiled, GLM53F_WI4M with levels and
 * steps int4 MFMA-tiled) [rows][cols/2] packed
 * levels and [rows][scols] steps. */
static int mat_i4(const Glm53fMat *m) { return m->dt == GLM53F_WI4 || m->dt == GLM53F_WI4T || m->dt == GLM53F_WI4M; }
static size_t mat_code_bytes(const Glm53fMat *m)
{
    return mat_i4(m) ? (size_t)m->rows * (size_t)(m->cols / 2) : (size_t)m->rows * (size_t)m->cols;
}
static size_t mat_scale_bytes(const Glm53fMat *m)
{
    const size_t srows = mat_i4(m) ? (size_t)m->rows : (size_t)((m->rows + m->br - 1) / m->br);
    return srows * (size_t)m->scols * sizeof(float);
}
static int mat_flags(const Glm53fMat *m)
{
    return m->dt == GLM53F_WF8T ? G53H_MAT_TILED : m->dt == GLM53F_WF8M ? G53H_MAT_MTILED
           : m->dt == GLM53F_WI4 ? G53H_MAT_I4 : m->dt == GLM53F_WI4T ? (G53H_MAT_I4 | G53H_MAT_I4T)
           : m->dt == GLM53F_WI4M ? (G53H_MAT_I4 | G53H_MAT_MTILED) : 0;
}

static void check_f8(const Glm53fMat *m, const char *what)
{
    if (!m->w) { fprintf(stderr, "glm53f: FATAL, multiply through an unbound matrix (%s)\n", what); abort(); }
    if (m->dt != GLM53F_WF8 && m->dt != GLM53F_WF8T && m->dt != GLM53F_WF8M && !mat_i4(m)) {
        fprintf(stderr, "glm53f: FATAL, %s has storage type %d; the MI355X expert path multiplies "
                        "FP8 E4M3 and int4 (GLM53F_WI4) matrices only\n", what, m->dt);
        abort();
    }
    if (mat_i4(m) && (m->cols & 1)) {
        fprintf(stderr, "glm53f: FATAL, %s is int4 with %d columns (two levels per byte need an even count)\n",
                what, m->cols);
        abort();
    }
    if (m->br <= 0 || m->bc <= 0 || m->scols != (m->cols + m->bc - 1) / m->bc) {
        fprintf(stderr, "glm53f: FATAL, %s has block %dx%d and %d scale columns for %d columns\n",
                what, m->br, m->bc, m->scols, m->cols);
        abort();
    }
    if ((m->dt == GLM53F_WF8T || m->dt == GLM53F_WF8M) && (m->rows % 8 || m->cols % 128)) {
        fprintf(stderr, "glm53f: FATAL, %s is tiled with %d rows and %d columns (rows a multiple of 8, "
                        "columns of 128)\n", what, m->rows, m->cols);
        abort();
    }
}

static void check_rowmajor(const Glm53fMat *m, const char *what)
{
    check_f8(m, what);
    if (m->dt == GLM53F_WF8T || m->dt == GLM53F_WF8M) {
        fprintf(stderr, "glm53f: FATAL, %s is tiled; layer weights are bound row-major (GLM53F_WF8)\n", what);
        abort();
    }
}

static G53hMat dev_mat_resident(const Glm53fMat *m, const char *what)
{
    check_rowmajor(m, what);
    G53hMat d;
    memset(&d, 0, sizeof d);
    d.w = (const uint8_t *)resident(m->w, mat_code_bytes(m));
    d.s = (const float *)resident(m->s, mat_scale_bytes(m));
    d.rows = m->rows; d.cols = m->cols; d.br = m->br; d.bc = m->bc; d.scols = m->scols;
    d.flags = mat_flags(m);
    return d;
}

static G53hMat view_mat_f8(const Glm53fMat *m)
{
    G53hMat d;
    memset(&d, 0, sizeof d);
    d.w = (const uint8_t *)m->w; d.s = m->s;
    d.rows = m->rows; d.cols = m->cols; d.br = m->br; d.bc = m->bc; d.scols = m->scols;
    d.flags = mat_flags(m);
    return d;
}

/* ---------------------------------------------------------- staging buffers ---- */
typedef struct { void *d; size_t n; } G53Buf;

static void *buf_get(G53Buf *b, size_t n)
{
    if (n <= b->n) return b->d;
    if (b->d && (g53h_sync() || g53h_free(b->d))) g53_die("freeing a staging buffer");
    b->d = g53h_alloc(n);
    if (!b->d) g53_die("allocating a staging buffer");
    b->n = n;
    return b->d;
}

static G53Buf g_xin, g_out, g_idx, g_w, g_flag, g_table, g_pred, g_tmp, g_contrib;

/* The same in the octet-tiled layout (for the tiled decode kernel), resident as well: uploaded
 * row-major once, converted on the device, kept under the host address with its own tag. */
static G53Buf g_tile_stage;
/* mfma != 0: the MFMA-tiled copy (G53H_MAT_MTILED) instead of the octet-tiled one; each layout
 * is kept under its own key. */
static G53hMat dev_mat_resident_tiled_as(const Glm53fMat *m, const char *what, int mfma)
{
    check_rowmajor(m, what);
    if (m->dt != GLM53F_WF8) {
        fprintf(stderr, "glm53f: FATAL, %s: only FP8 matrices are kept tiled\n", what);
        abort();
    }
    G53hMat d;
    memset(&d, 0, sizeof d);
    d.rows = m->rows; d.cols = m->cols; d.br = m->br; d.bc = m->bc; d.scols = m->scols;
    d.flags = mfma ? G53H_MAT_MTILED : G53H_MAT_TILED;
    d.s = (const float *)resident(m->s, mat_scale_bytes(m));
    if (g53h_is_device_ptr(m->w)) {
        fprintf(stderr, "glm53f: FATAL, %s: an HBM matrix is used as it is, not converted\n", what);
        abort();
    }
    const size_t n = mat_code_bytes(m);
    const char *key = (const char *)m->w + (mfma ? 2 : 1); /* the tiled copy's own key */
    const int rdt = mfma ? -3 : -2;
    G53Res *r = res_find(key);
    if (r && r->n == n && r->dt == rdt && res_same(r, m->w, n)) { d.w = (const uint8_t *)r->d; return d; }
    uint8_t *stage = (uint8_t *)buf_get(&g_tile_stage, n);
    uint8_t *t = (uint8_t *)g53h_alloc(n);
    if (!t || g53h_h2d(stage, m->w, n) ||
        (mfma ? g53h_mtile_f8(t, stage, m->rows, m->cols, 0) : g53h_tile_f8(t, stage, m->rows, m->cols)) || g53h_sync())
        g53_die("tiling a resident weight");
    if (!r) r = res_insert(key);
    else if (g53h_sync() || g53h_free(r->d)) g53_die("replacing a resident weight");
    r->n = n; r->d = t; r->dt = rdt;
    res_record(r, m->w, n);
    d.w = t;
    return d;
}
static G53hMat dev_mat_resident_tiled(const Glm53fMat *m, const char *what)
{
    return dev_mat_resident_tiled_as(m, what, 0);
}

/* Host operand -> HBM (or the operand itself when it is HBM already). */
static const float *stage_in(G53Buf *b, const float *h, size_t n)
{
    if (g53h_is_device_ptr(h)) return h;
    float *d = (float *)buf_get(b, n * sizeof(float));
    if (g53h_h2d(d, h, n * sizeof(float))) g53_die("staging an operand");
    return d;
}

static void ensure_device(void)
{
    if (g53h_init(0)) g53_die("initialising the GPU");
}

/* ------------------------------------------------------------ unit operations ---- */
float glm53f_e4m3f(uint8_t b) { return g53_e4m3_to_f32(b); }

/* A matrix passed to the unit operations is copied per call (its memory may be reused by the
 * caller for another matrix); MoE weights are the ones kept resident. */
static G53Buf g_mat[3];
static G53hMat dev_mat_staged(const Glm53fMat *m, G53Buf *b, const char *what)
{
    check_f8(m, what);
    if (m->dt == GLM53F_WI4T || m->dt == GLM53F_WI4M || m->dt == GLM53F_WF8M) {
        fprintf(stderr, "glm53f: FATAL, %s is a tiled cache view (GLM53F_WI4T / GLM53F_WI4M / GLM53F_WF8M); "
                        "only glm53f_moe reads those\n", what);
        abort();
    }
    const int dev = g53h_is_device_ptr(m->w);
    if (dev && m->dt != GLM53F_WF8T) return view_mat_f8(m);
    const size_t cb = mat_code_bytes(m), sb = mat_scale_bytes(m);
    uint8_t *d = (uint8_t *)buf_get(b, ((cb + 255) & ~(size_t)255) + sb);
    G53hMat r = view_mat_f8(m);
    if (m->dt == GLM53F_WF8T) {                      /* the unit kernels read row-major codes */
        const uint8_t *src = (const uint8_t *)m->w;
        if (!dev) {
            uint8_t *t = (uint8_t *)buf_get(&g_tile_stage, cb);
            if (g53h_h2d(t, m->w, cb)) g53_die(what);
            src = t;
        }
        if (g53h_untile_f8(d, src, m->rows, m->cols)) g53_die(what);
        r.flags = 0;
    } else if (g53h_h2d(d, m->w, cb)) {
        g53_die(what);
    }
    if (dev) {
        r.w = d;
        return r;
    }
    if (g53h_h2d(d + ((cb + 255) & ~(size_t)255), m->s, sb)) g53_die(what);
    r.w = d;
    r.s = (const float *)(d + ((cb + 255) & ~(size_t)255));
    return r;
}

void glm53f_mm_batch(float *y, const float *x, int T, const Glm53fMat *m)
{
    if (T < 1) return;
    ensure_device();
    const G53hMat d = dev_mat_staged(m, &g_mat[0], "glm53f_mm");
    const float *xd = stage_in(&g_xin, x, (size_t)T * m->cols);
    const int yd_dev = g53h_is_device_ptr(y);
    float *yd = yd_dev ? y : (float *)buf_get(&g_out, (size_t)T * m->rows * sizeof(float));
    if (g53h_mm_f8(yd, xd, T, &d)) g53_die("glm53f_mm");
    if (!yd_dev && g53h_d2h(y, yd, (size_t)T * m->rows * sizeof(float))) g53_die("glm53f_mm");
    if (yd_dev && g53h_sync()) g53_die("glm53f_mm");
}

void glm53f_mm(float *y, const float *x, const Glm53fMat *m) { glm53f_mm_batch(y, x, 1, m); }

void glm53f_i4_from_f8(unsigned char *q, float *steps, const Glm53fMat *src)
{
    ensure_device();
    check_f8(src, "glm53f_i4_from_f8");
    if (mat_i4(src) || src->cols % GLM53F_I4_GROUP) {
        fprintf(stderr, "glm53f: FATAL, glm53f_i4_from_f8 needs an FP8 matrix with columns a multiple of %d\n",
                GLM53F_I4_GROUP);
        abort();
    }
    const G53hMat d = dev_mat_staged(src, &g_mat[0], "glm53f_i4_from_f8");
    const size_t qb = (size_t)src->rows * (size_t)(src->cols / 2);
    const size_t sb = (size_t)src->rows * (size_t)(src->cols / GLM53F_I4_GROUP) * sizeof(float);
    const int qdev = g53h_is_device_ptr(q), sdev = g53h_is_device_ptr(steps);
    uint8_t *qd = qdev ? q : (uint8_t *)buf_get(&g_mat[1], qb);
    float *sd = sdev ? steps : (float *)buf_get(&g_mat[2], sb);
    if (g53h_i4_from_f8(qd, sd, &d)) g53_die("glm53f_i4_from_f8");
    if ((!qdev && g53h_d2h(q, qd, qb)) || (!sdev && g53h_d2h(steps, sd, sb)) || g53h_sync())
        g53_die("glm53f_i4_from_f8");
}

void glm53f_swiglu_clamp(float *y, const float *gu, int n, float limit)
{
    if (n < 1) return;
    ensure_device();
    const float *gd = stage_in(&g_xin, gu, (size_t)2 * n);
    const int ydev = g53h_is_device_ptr(y);
    float *yd = ydev ? y : (float *)buf_get(&g_out, (size_t)n * sizeof(float));
    if (g53h_swiglu(yd, gd, n, 1, limit)) g53_die("glm53f_swiglu_clamp");
    if (!ydev && g53h_d2h(y, yd, (size_t)n * sizeof(float))) g53_die("glm53f_swiglu_clamp");
    if (ydev && g53h_sync()) g53_die("glm53f_swiglu_clamp");
}

size_t glm53f_mlp_scratch(const Glm53fCfg *c)
{
    const int I = c->dense_inter > c->moe_inter * c->n_shared ? c->dense_inter : c->moe_inter * c->n_shared;
    return (size_t)3 * I;
}

void glm53f_mlp(float *out, const float *x, const Glm53fMat *gate, const Glm53fMat *up,
                const Glm53fMat *down, float limit, float *scratch)
{
    (void)scratch;
    ensure_device();
    const G53hMat g = dev_mat_staged(gate, &g_mat[0], "mlp gate"), u = dev_mat_staged(up, &g_mat[1], "mlp up");
    const G53hMat dn = dev_mat_staged(down, &g_mat[2], "mlp down");
    const int I = gate->rows, E = down->rows;
    const float *xd = stage_in(&g_xin, x, (size_t)gate->cols);
    float *tmp = (float *)buf_get(&g_tmp, (size_t)3 * I * sizeof(float));
    const int odev = g53h_is_device_ptr(out);
    float *od = odev ? out : (float *)buf_get(&g_out, (size_t)E * sizeof(float));
    if (g53h_mm_f8(tmp, xd, 1, &g) || g53h_mm_f8(tmp + I, xd, 1, &u) ||
        g53h_swiglu(tmp + 2 * I, tmp, I, 1, limit) || g53h_mm_f8(od, tmp + 2 * I, 1, &dn))
        g53_die("glm53f_mlp");
    if (!odev && g53h_d2h(out, od, (size_t)E * sizeof(float))) g53_die("glm53f_mlp");
    if (odev && g53h_sync()) g53_die("glm53f_mlp");
}

/* ------------------------------------------------------------------ router ---- */
static void route_dev(int *idx_d, float *w_d, const float *xd, int T, const Glm53fMoeW *m,
                      const Glm53fCfg *c)
{
    int dt = 0;
    const void *gate = resident_router(m->gate, (size_t)c->n_experts * c->hidden, &dt);
    const float *bias = (const float *)resident(m->bias, (size_t)c->n_experts * sizeof(float));
    int *flag = (int *)buf_get(&g_flag, 256);
    if (g53h_memset(flag, 0, sizeof(int)) ||
        g53h_router(idx_d, w_d, xd, T, gate, dt, bias, c->n_experts, c->hidden, c->topk, c->norm_topk,
                    c->routed_scale, flag))
        g53_die("glm53f_router");
    int bad = 0;
    if (g53h_d2h(&bad, flag, sizeof bad)) g53_die("glm53f_router");
    if (bad) {
        fprintf(stderr, "glm53f: FATAL, router selection (NaN scores) found no candidate\n");
        abort();
    }
}

void glm53f_router(int *idx, float *w, const float *x, const Glm53fMoeW *m, const Glm53fCfg *c)
{
    ensure_device();
    if (c->n_experts > 1024) {
        fprintf(stderr, "glm53f: FATAL, routed experts is %d, above the limit of 1024.\n", c->n_experts);
        abort();
    }
    const int K = c->topk;
    const float *xd = stage_in(&g_xin, x, (size_t)c->hidden);
    int *idx_d = (int *)buf_get(&g_idx, (size_t)K * sizeof(int));
    float *w_d = (float *)buf_get(&g_w, (size_t)K * sizeof(float));
    route_dev(idx_d, w_d, xd, 1, m, c);
    if (g53h_d2h(idx, idx_d, (size_t)K * sizeof(int)) || g53h_d2h(w, w_d, (size_t)K * sizeof(float)))
        g53_die("glm53f_router");
}

/* ---------------------------------------------------------------------- MoE ---- */
size_t glm53f_moe_scratch(const Glm53fCfg *c, int T)
{
    const size_t n = (size_t)(T < G53_MOE_CHUNK ? T : G53_MOE_CHUNK);
    const size_t E = (size_t)c->hidden, K = (size_t)c->topk;
    return n * K * E + n * K * 2 + (size_t)3 * c->moe_inter + E + glm53f_mlp_scratch(c) + E +
           n * (2 * E + 3 * (size_t)c->moe_inter);
}

static void check_expert_shape(const Glm53fExpertQ *q, const Glm53fCfg *c, int layer, int e)
{
    const Glm53fMat *ms[3] = {&q->gate, &q->up, &q->down};
    const int rows[3] = {c->moe_inter, c->moe_inter, c->hidden}, cols[3] = {c->hidden, c->hidden, c->moe_inter};
    for (int i = 0; i < 3; i++) {
        check_f8(ms[i], "a routed expert matrix");
        if (ms[i]->rows != rows[i] || ms[i]->cols != cols[i]) {
            fprintf(stderr, "glm53f: FATAL, layer %d expert %d matrix %d is %dx%d, expected %dx%d\n",
                    layer, e, i, ms[i]->rows, ms[i]->cols, rows[i], cols[i]);
            abort();
        }
    }
}

static void *g_pin_x, *g_pin_tab, *g_pin_back, *g_pin_err;
static size_t g_pin_x_n, g_pin_tab_n, g_pin_back_n, g_pin_err_n;

static void *pinned(void **p, size_t *have, size_t n)
{
    if (n <= *have) return *p;
    if (*p && (g53h_sync() || g53h_host_free(*p))) g53_die("freeing pinned staging");
    *p = g53h_host_alloc(n);
    if (!*p) g53_die("allocating pinned staging");
    *have = n;
    return *p;
}

/* ------------------------------------------------------------- error flags ---- */
/* The layer kernels' flags come back with the layer's last copy (g53h_errors_async before it):
 * a wait that gave up or an unusable descriptor aborts, as the reference aborts on its own
 * errors (src/core/glm53f_ops.c:28-39); a token without K selectable experts is the reference's
 * NaN routing abort (:961-965). */
static int *errors_enqueue(void)
{
    int *e = (int *)pinned(&g_pin_err, &g_pin_err_n, G53H_NERR * sizeof(int));
    if (g53h_errors_async(e)) g53_die("reading the kernel error flags");
    return e;
}

static void errors_check(const int *e, int layer, int K)
{
    const int dec = e[0] | e[1], grp = e[2];
    if (dec & 2) {
        fprintf(stderr, "glm53f: FATAL, router selection (NaN scores) is below %d, above the limit of %d.\n", K, K);
        abort();
    }
    if (dec || grp) {
        fprintf(stderr, "glm53f: FATAL, the MoE kernels of layer %d reported error flags (decode 0x%x, grouped 0x%x):"
                        "%s%s%s; aborting rather than returning a corrupt output.\n",
                layer, dec, grp, ((dec | grp) & 1) ? " a bound or wait was exceeded" : "",
                (grp & 2) ? " a wait between waves timed out" : "",
                ((dec | grp) & 8) ? " an expert descriptor the kernels cannot read" : "");
        abort();
    }
}

/* --------------------------------------------------------- switches (env) ---- */
/* GLM53F_NO_PREFILL_PREFETCH and GLM53F_PREFILL_PRED, read once (src/core/glm53f_ops.c:1186-1194). */
static int g_prefill_off = -1, g_prefill_pred = -1;
static void read_switches(void)
{
    if (g_prefill_off >= 0) return;
    g_prefill_off = getenv("GLM53F_NO_PREFILL_PREFETCH") ? 1 : 0;
    const char *pp = getenv("GLM53F_PREFILL_PRED");
    g_prefill_pred = pp ? atoi(pp) : -1;
}

/* GLM53F_ROUTE_TOP16=path: one line per decode MoE layer, the 16 best candidates in selection
 * order as id:score (the sigmoid before normalisation), the format of the reference's
 * route_top16_trace (src/core/glm53f_ops.c:1044-1080), from the device router. */
static FILE *g_top16 = NULL;
static int g_top16_on = -1;
static void route_top16(int layer, const float *xd, const Glm53fMoeW *w, const Glm53fCfg *c)
{
    if (g_top16_on < 0) {
        const char *p = getenv("GLM53F_ROUTE_TOP16");
        g_top16 = p ? fopen(p, "a") : NULL;
        g_top16_on = g_top16 != NULL;
    }
    if (!g_top16_on) return;
    const int NE = c->n_experts, n = NE < 16 ? NE : 16;
    int dt = 0;
    const void *gate = resident_router(w->gate, (size_t)NE * c->hidden, &dt);
    const float *bias = (const float *)resident(w->bias, (size_t)NE * sizeof(float));
    int *id_d = (int *)buf_get(&g_tmp, 32 * sizeof(int));
    float *sc_d = (float *)(id_d + 16);
    int ids[16];
    float sc[16];
    if (g53h_route_topn_batch(id_d, sc_d, n, xd, 1, gate, dt, bias, NE, c->hidden) ||
        g53h_d2h(ids, id_d, (size_t)n * sizeof(int)) || g53h_d2h(sc, sc_d, (size_t)n * sizeof(float)))
        g53_die("the routing trace");
    fprintf(g_top16, "%d", layer);
    for (int j = 0; j < n; j++) fprintf(g_top16, " %d:%.6g", ids[j], sc[j]);
    fputc('\n', g_top16);
    fflush(g_top16);
}

/* ------------------------------------------------------- next-layer prediction ---- */
/* The experts layer + 1 will probably want, for the hint protocol (src/core/glm53f_ops.c:
 * 1021-1042, 1196-1226): at T = 1 the next router's top `per` on this input; for a chunk of
 * tokens every token's top `per`, merged by the device vote (most voted first, ties in order of
 * first appearance). All tokens in one launch, one copy back. Returns the count written. */
static int predict_next(int *pred, const float *xd, const Glm53fMoeW *w, const Glm53fCfg *c, int T, int per)
{
    const int NE = c->n_experts, E = c->hidden;
    int dt = 0;
    const void *gate = resident_router(w->next_gate, (size_t)NE * E, &dt);
    const float *bias = (const float *)resident(w->next_bias, (size_t)NE * sizeof(float));
    int *ids_d = (int *)buf_get(&g_pred, ((size_t)T * per + 1 + NE) * sizeof(int));
    if (g53h_route_topn_batch(ids_d, NULL, per, xd, T, gate, dt, bias, NE, E)) g53_die("next-layer prediction");
    if (T == 1) {
        if (g53h_d2h(pred, ids_d, (size_t)per * sizeof(int))) g53_die("next-layer prediction");
        return per;
    }
    int *vote_d = ids_d + (size_t)T * per;
    if (g53h_vote(vote_d, ids_d, T, per, NE)) g53_die("next-layer prediction");
    int *back = (int *)pinned(&g_pin_back, &g_pin_back_n, (size_t)(1 + NE) * sizeof(int));
    if (g53h_d2h(back, vote_d, (size_t)(1 + NE) * sizeof(int))) g53_die("next-layer prediction");
    const int no = back[0] < 64 * 2 * GLM53F_MAX_TOPK ? back[0] : 64 * 2 * GLM53F_MAX_TOPK;
    memcpy(pred, back + 1, (size_t)no * sizeof(int));
    return no;
}

/* --------------------------------------------------- decode through the HBM cache ---- */
/* One token with the experts served by this library's HBM cache, in one fused launch: the
 * reference's protocol (route, hint the own then the next layer's experts, get, multiply,
 * release; src/core/glm53f_ops.c:1169-1342) with two host round trips. The routing, the
 * prediction and the NaN flag come back in one copy; an expert that fails to load is the
 * reference's drop (counted, reported, its contribution zero). With octet-tiled slots the layer
 * kernel takes the routing as given (it is not computed twice) and a compact table of the K
 * chosen descriptors and the shared one (K + 1 descriptors uploaded); with row-major slots it
 * routes again with the same bit-exact router, over a table that holds only the chosen ones. */
static G53Buf g_ident;

/* Mailbox use of the cached decode: slot 0 carries the routing read-back (idx, flag, prediction
 * at byte 1024), slot 1 the error flags and the output (at byte 4096). */
#define G53_MB_ROUTE 0
#define G53_MB_ROUTE_OFF 1024
#define G53_MB_OUT 1
#define G53_MB_OUT_OFF 4100                 /* the output after the 3 error words: 16-byte aligned */
static unsigned g_seq;
static unsigned next_seq(void)
{
    if (++g_seq == 0) g_seq = 1;                     /* 0 is the mailbox's initial value */
    return g_seq;
}

#ifdef G53_HOST_PROF
#include <time.h>
static double g_hp[16];
static long g_hp_n;
static double hp_now(void) { struct timespec t; clock_gettime(CLOCK_MONOTONIC, &t); return t.tv_sec * 1e6 + t.tv_nsec * 1e-3; }
#define HP(i) do { const double t_ = hp_now(); g_hp[i] += t_ - hp_t; hp_t = t_; } while (0)
void g53h_host_prof(double *out) { for (int i = 0; i < 16; i++) out[i] = g_hp_n ? g_hp[i] / g_hp_n : 0; memset(g_hp, 0, sizeof g_hp); g_hp_n = 0; }
#else
#define HP(i) do { } while (0)
#endif

/* The shared expert can be kept octet-tiled: FP8 with 128-column blocks, whole row octets. */
static int shared_tileable(const Glm53fMoeW *w)
{
    const Glm53fMat *ms[3] = {&w->sh_gate, &w->sh_up, &w->sh_down};
    for (int i = 0; i < 3; i++)
        if (ms[i]->dt != GLM53F_WF8 || ms[i]->bc != 128 || ms[i]->rows % 8 || ms[i]->cols % 128) return 0;
    return 1;
}

/* G53H_NO_SPECULATE (set at the first call) turns the speculative cached layer off: every layer
 * then routes first and fetches before it computes (a switch of this library, for comparisons). */
static int g_spec = -1;
static int spec_enabled(void)
{
    if (g_spec < 0) g_spec = getenv("G53H_NO_SPECULATE") ? 0 : 1;
    return g_spec;
}
static int64_t g_spec_n[3];     /* layers: speculative and done, speculative and run again, not */
/* The last 16 speculative layers' outcomes (bit set: finished by the speculative launch). A
 * layer speculates while at least half of them finished, and every 16th layer regardless, so
 * that a cache that misses most of the time (a small budget) pays for few wasted launches. */
static unsigned g_spec_hist = 0xffffu, g_spec_tick = 0;
static int spec_worth(void)
{
    return __builtin_popcount(g_spec_hist & 0xffffu) >= 8 || (++g_spec_tick & 15) == 0;
}
static void spec_outcome(int done) { g_spec_hist = (g_spec_hist << 1) | (done ? 1u : 0u); }
void g53h_speculate_counts(int64_t *out)
{
    for (int i = 0; i < 3; i++) { out[i] = g_spec_n[i]; g_spec_n[i] = 0; }
}
int g53h_set_speculate(int on)
{
    const int prev = spec_enabled();
    g_spec = on ? 1 : 0;
    g_spec_hist = 0xffffu;          /* a fresh history: the next layers speculate */
    g_spec_tick = 0;
    return prev;
}

/* The shared expert's descriptor in HBM (octet-tiled, or MFMA-tiled when mfma != 0; resident),
 * one per layer and layout, uploaded when it changes. */
static G53hExpert g_shh[2][GLM53F_MAX_LAYERS + 1];
static G53Buf g_shd[2];
static const G53hExpert *shared_desc(const Glm53fMoeW *w, int mfma)
{
    const int l = w->layer >= 0 && w->layer <= GLM53F_MAX_LAYERS ? w->layer : GLM53F_MAX_LAYERS;
    const int k = mfma ? 1 : 0;
    G53hExpert *d = (G53hExpert *)buf_get(&g_shd[k], (size_t)(GLM53F_MAX_LAYERS + 1) * sizeof(G53hExpert));
    G53hExpert e;
    memset(&e, 0, sizeof e);
    e.gate = dev_mat_resident_tiled_as(&w->sh_gate, "shared gate", k);
    e.up = dev_mat_resident_tiled_as(&w->sh_up, "shared up", k);
    e.down = dev_mat_resident_tiled_as(&w->sh_down, "shared down", k);
    if (memcmp(&e, &g_shh[k][l], sizeof e)) {
        g_shh[k][l] = e;
        if (g53h_h2d_async(d + l, &g_shh[k][l], sizeof e)) g53_die("glm53f_moe");
    }
    return d + l;
}

/* x (host memory) into xd without a wait: through the mapped inbox, read by a kernel on the
 * compute stream (the previous call's fetch has run: its output was waited for), or a copy from
 * pinned staging when it does not fit the inbox. */
static void upload_x(float *xd, const float *x, int E)
{
    const size_t xb = (size_t)E * sizeof(float);
    if (xb <= G53H_INBOX_BYTES && xb % 16 == 0) {
        memcpy(g53h_inbox(), x, xb);
        if (g53h_inbox_fetch(xd, 0, xb)) g53_die("glm53f_moe");
    } else {
        float *xp = (float *)pinned(&g_pin_x, &g_pin_x_n, xb);
        memcpy(xp, x, xb);
        if (g53h_h2d_async(xd, xp, xb)) g53_die("glm53f_moe");
    }
}

static void decode_cached(float *out, const float *x, const Glm53fMoeW *w, const Glm53fCfg *c, int with_shared)
{
    const int E = c->hidden, K = c->topk, NE = c->n_experts;
    Glm53fExpertSrc *src = w->src;
#ifdef G53_HOST_PROF
    double hp_t = hp_now();
    g_hp_n++;
#endif
    /* x goes up right before the first launch that reads it (upload_x below), after the host's
     * preparation, so that the layer kernel's launch follows the fetch closely */
    float *xd = (float *)x;
    const int x_host = !g53h_is_device_ptr(x);
    if (x_host) xd = (float *)buf_get(&g_xin, (size_t)E * sizeof(float));
    HP(8);
    const int per_max = 2 * GLM53F_MAX_TOPK;
    int *rd = (int *)buf_get(&g_idx, (size_t)(K + 1 + per_max) * sizeof(int));
    int *idx_d = rd, *flag_d = rd + K, *pred_d = rd + K + 1;
    float *w_d = (float *)buf_get(&g_w, (size_t)K * sizeof(float));
    int dt = 0, ndt = 0;
    HP(10);
    const void *gate = resident_router(w->gate, (size_t)NE * E, &dt);
    HP(11);
    const float *bias = (const float *)resident(w->bias, (size_t)NE * sizeof(float));
    HP(12);
    const int prefetch = w->prefetch_n > 0 && src->hint != NULL;
    int per = 0;
    const void *ngate = NULL;
    const float *nbias = NULL;
    if (prefetch && w->next_gate) {
        per = w->prefetch_n < per_max ? w->prefetch_n : per_max;
        if (per > NE) per = NE;
        ngate = resident_router(w->next_gate, (size_t)NE * E, &ndt);
        HP(13);
        nbias = (const float *)resident(w->next_bias, (size_t)NE * sizeof(float));
    }
    HP(9);
    const int odev = g53h_is_device_ptr(out);
    float *od = odev ? out : (float *)buf_get(&g_out, (size_t)E * sizeof(float));
    const size_t ob = odev ? 0 : (size_t)E * sizeof(float);
    /* Speculative layer: with the HBM cache's octet-tiled slots, the one-launch decode routes by
     * itself over the table of this layer's landed slots, the next layer's prediction and the
     * mailbox copy follow, and the host waits once. The reference's calls (hints, gets, releases)
     * are then made in its order on the routing that came back; if a chosen expert had no landed
     * slot at the launch (its contribution was left out) or a get fails, the layer is run again
     * below on the experts the gets returned. No cache call happens while the kernel runs, so
     * no slot it reads is refilled under it. */
    const G53hExpert *stab_d = NULL, *stab_h = NULL;
    /* 1 octet-tiled FP8 slots, 2 MFMA-tiled FP8, 3 int4-tiled, 4 int4 MFMA-tiled */
    const int kind = g53h_cache_slot_kind(src);
    int spec = spec_enabled() && spec_worth() && dt == 1 && K <= 15 && NE <= 1024 && E == 4096 && c->moe_inter == 2048 &&
               G53_MB_OUT_OFF + 4 * G53H_NERR + ob <= G53H_MBOX_BYTES &&
               (!with_shared || shared_tileable(w)) && g53h_cache_layer_table(src, w->layer, &stab_d, &stab_h) == 0;
    const int *back;
    const int spec_launched = spec;
    if (spec) {
        G53hMoeLayer SL;
        memset(&SL, 0, sizeof SL);
        SL.hidden = E; SL.inter = c->moe_inter; SL.topk = K; SL.norm_topk = c->norm_topk;
        SL.routed_scale = c->routed_scale; SL.swiglu_limit = c->swiglu_limit;
        SL.router = gate; SL.router_dt = dt; SL.bias = bias; SL.block_c = 128; SL.tiled = kind >= 2 && kind <= 4 ? kind : 1;
        SL.n_experts = NE; SL.experts = stab_d;
        SL.shared = with_shared ? shared_desc(w, kind == 2 || kind == 4) : NULL;
        HP(7);
        if (x_host) upload_x(xd, x, E);
        if (per > 0 && g53h_decode_next(xd, ngate, ndt, nbias, NE, E)) g53_die("glm53f_router");
        HP(14);
        if (g53h_moe(od, xd, 1, &SL, idx_d, w_d)) g53_die("glm53f_moe");
        HP(15);
        const unsigned seq_s = next_seq();
        if (g53h_decode_publish(G53_MB_OUT, seq_s, G53_MB_ROUTE_OFF, idx_d, K, pred_d, per, NE, G53_MB_OUT_OFF, od, ob))
            g53_die("glm53f_moe");
        HP(0);
        if (g53h_mailbox_wait(G53_MB_OUT, seq_s)) g53_die("glm53f_moe");
        HP(1);
        back = (const int *)((const char *)g53h_mailbox() + G53_MB_ROUTE_OFF);
    } else {
        /* routing, NaN flag and the next layer's prediction: two launches, and the kernel writes
         * the host's copy into the mailbox, which the host polls */
        const unsigned seq_r = next_seq();
        if (x_host) upload_x(xd, x, E);
        if (g53h_route_decode(idx_d, w_d, flag_d, pred_d, per, xd, gate, dt, bias, ngate, ndt, nbias, NE, E, K,
                              c->norm_topk, c->routed_scale, G53_MB_ROUTE, seq_r, G53_MB_ROUTE_OFF))
            g53_die("glm53f_router");
        HP(0);
        if (g53h_mailbox_wait(G53_MB_ROUTE, seq_r)) g53_die("glm53f_moe routing");
        back = (const int *)((const char *)g53h_mailbox() + G53_MB_ROUTE_OFF);
        HP(1);
    }
    if (back[K]) {
        fprintf(stderr, "glm53f: FATAL, router selection (NaN scores) is below %d, above the limit of %d.\n", K, K);
        abort();
    }
    int ids[GLM53F_MAX_TOPK];
    memcpy(ids, back, (size_t)K * sizeof(int));
    if (spec) {
        /* the layer's flags (the routing's NaN case is handled above, as the reference's) */
        errors_check((const int *)((const char *)g53h_mailbox() + G53_MB_OUT_OFF), w->layer, K);
        /* the table is as it was at the launch: no cache call since */
        for (int j = 0; j < K; j++)
            if (ids[j] < 0 || ids[j] >= NE || !stab_h[ids[j]].gate.w) spec = 0;
    }
    route_top16(w->layer, xd, w, c);
    if (prefetch) {
        src->hint(src, w->layer, ids, K);
        if (per > 0) src->hint(src, w->layer + 1, back + K + 1, per);
    }
    HP(2);
    /* the chosen experts' views (slot order), the shared expert after them */
    G53hExpert *tab = (G53hExpert *)pinned(&g_pin_tab, &g_pin_tab_n, (size_t)(NE + 1) * sizeof(G53hExpert));
    int held[GLM53F_MAX_TOPK], nh = 0, tiled = 1, mt = 1, i4r = 1, i4t = 1, i4m = 1;
    memset(tab, 0, (size_t)(K + 1) * sizeof(G53hExpert));
    for (int j = 0; j < K; j++) {
        Glm53fExpertQ q;
        memset(&q, 0, sizeof q);
        if (src->get(src, w->layer, ids[j], &q) != 0) {
            spec = 0;                              /* the speculative output included it */
            glm53f_expert_drops++;
            fprintf(stderr, "EXPERT DROP: layer %d expert %d failed to load; this output is CORRUPT\n", w->layer,
                    ids[j]);
            tab[j].gate.flags = G53H_MAT_DROPPED;  /* its contribution is zero */
            continue;
        }
        held[nh++] = ids[j];
        check_expert_shape(&q, c, w->layer, ids[j]);
        tab[j].gate = view_mat_f8(&q.gate);
        tab[j].up = view_mat_f8(&q.up);
        tab[j].down = view_mat_f8(&q.down);
        if (!(tab[j].gate.flags & tab[j].up.flags & tab[j].down.flags & G53H_MAT_TILED)) tiled = 0;
        if (((tab[j].gate.flags | tab[j].up.flags | tab[j].down.flags) & G53H_MAT_I4) ||
            !(tab[j].gate.flags & tab[j].up.flags & tab[j].down.flags & G53H_MAT_MTILED))
            mt = 0;
        if (!(tab[j].gate.flags & tab[j].up.flags & tab[j].down.flags & G53H_MAT_I4)) i4r = 0;
        if (!(tab[j].gate.flags & tab[j].up.flags & tab[j].down.flags & G53H_MAT_I4T)) i4t = 0;
        if (!(tab[j].gate.flags & tab[j].up.flags & tab[j].down.flags & G53H_MAT_I4) ||
            !(tab[j].gate.flags & tab[j].up.flags & tab[j].down.flags & G53H_MAT_MTILED))
            i4m = 0;
    }
    if (!nh) i4r = i4t = i4m = mt = 0;
    HP(3);
    if (spec) {                  /* every chosen expert was in the kernel's table: the output is done */
        g_spec_n[0]++;
        spec_outcome(1);
        for (int i = 0; i < nh; i++) src->release(src, w->layer, held[i]);
        if (ob) memcpy(out, (const char *)g53h_mailbox() + G53_MB_OUT_OFF + 4 * G53H_NERR, ob);
        HP(6);
        return;
    }
    g_spec_n[spec_launched ? 1 : 2]++;
    if (spec_launched) spec_outcome(0);
    if (with_shared) {
        /* the shared expert resident in the layout of the routed slots */
        /* (int4 routed experts: the row-wave kernel's fast FP8 path reads it octet-tiled too) */
        const int tile_ok = (tiled || mt || i4r) && shared_tileable(w);
        if (tile_ok) {           /* MFMA-tiled beside MFMA-tiled views, else octet-tiled */
            tab[K].gate = dev_mat_resident_tiled_as(&w->sh_gate, "shared gate", i4m || mt);
            tab[K].up = dev_mat_resident_tiled_as(&w->sh_up, "shared up", i4m || mt);
            tab[K].down = dev_mat_resident_tiled_as(&w->sh_down, "shared down", i4m || mt);
        } else {
            tab[K].gate = dev_mat_resident(&w->sh_gate, "shared gate");
            tab[K].up = dev_mat_resident(&w->sh_up, "shared up");
            tab[K].down = dev_mat_resident(&w->sh_down, "shared down");
            tiled = 0;
            mt = 0;
        }
        if (i4r) tiled = 0;
    }
    /* int4-tiled views: the one-launch int4 decode when the shared expert is octet-tiled (or
     * absent); else their levels untiled for the row kernels */
    const int one_i4t = i4t && (!with_shared || (tab[K].gate.flags & G53H_MAT_TILED));
    const int one_i4m = i4m && (!with_shared || (tab[K].gate.flags & G53H_MAT_MTILED));
    const int one_mt = mt && (!with_shared || (tab[K].gate.flags & G53H_MAT_MTILED));
    if ((i4t && !one_i4t) || (i4m && !one_i4m)) {
        /* the row kernels read row-major levels (and steps) */
        static G53Buf g_i4u[GLM53F_MAX_TOPK];
        for (int j = 0; j < K; j++) {
            G53hMat *ms[3] = {&tab[j].gate, &tab[j].up, &tab[j].down};
            if (!ms[0]->w) continue;
            size_t need = 0;
            for (int i = 0; i < 3; i++)
                need += ((((size_t)ms[i]->rows * (ms[i]->cols / 2)) + 255) & ~(size_t)255) +
                        (i4m ? (((size_t)ms[i]->rows * ms[i]->scols * 4 + 255) & ~(size_t)255) : 0);
            uint8_t *b = (uint8_t *)buf_get(&g_i4u[j], need);
            for (int i = 0; i < 3; i++) {
                uint8_t *lv = b;
                b += (((size_t)ms[i]->rows * (ms[i]->cols / 2)) + 255) & ~(size_t)255;
                if (i4m) {
                    float *st = (float *)b;
                    b += ((size_t)ms[i]->rows * ms[i]->scols * 4 + 255) & ~(size_t)255;
                    if (g53h_mtile_i4(lv, st, ms[i]->w, ms[i]->s, ms[i]->rows, ms[i]->cols, 1))
                        g53_die("converting an int4 expert view");
                    ms[i]->s = st;
                } else if (g53h_tile_i4(lv, ms[i]->w, ms[i]->rows, ms[i]->cols, 1)) {
                    g53_die("converting an int4 expert view");
                }
                ms[i]->w = lv;
                ms[i]->flags = G53H_MAT_I4;
            }
        }
    }
    G53hMoeLayer L;
    memset(&L, 0, sizeof L);
    L.hidden = E; L.inter = c->moe_inter; L.topk = K; L.norm_topk = c->norm_topk;
    L.routed_scale = c->routed_scale; L.swiglu_limit = c->swiglu_limit;
    L.router = gate; L.router_dt = dt; L.bias = bias; L.block_c = 128;
    for (int j = 0; j <= K; j++) {
        const G53hExpert *e = &tab[j];
        if ((j < K || with_shared) && e->gate.w && (e->gate.bc != 128 || e->up.bc != 128 || e->down.bc != 128 ||
                                                    ((e->gate.flags | e->up.flags | e->down.flags) & G53H_MAT_I4)))
            L.block_c = 0;
    }
    G53hExpert *tab_d = (G53hExpert *)buf_get(&g_table, (size_t)(NE + 1) * sizeof(G53hExpert));
    if (tiled || one_mt || one_i4t || one_i4m) {
        /* compact table: slot j holds the j-th chosen expert (the kernel is told indices 0 .. K-1),
         * slot K the shared expert */
        int *ident = (int *)buf_get(&g_ident, GLM53F_MAX_TOPK * sizeof(int));
        static int ident_ready = 0;
        if (!ident_ready) {
            int h[GLM53F_MAX_TOPK];
            for (int j = 0; j < GLM53F_MAX_TOPK; j++) h[j] = j;
            if (g53h_h2d(ident, h, sizeof h)) g53_die("glm53f_moe");
            ident_ready = 1;
        }
        if (g53h_h2d_async(tab_d, tab, (size_t)(K + 1) * sizeof(G53hExpert))) g53_die("glm53f_moe");
        L.n_experts = K; L.experts = tab_d; L.shared = with_shared ? tab_d + K : NULL;
        L.tiled = one_i4m ? 4 : one_i4t ? 3 : one_mt ? 2 : 1;
        L.block_c = 128;
        if (g53h_moe_routed_given(od, xd, 1, &L, ident, w_d)) g53_die("glm53f_moe");
    } else {
        /* the table indexed by expert: the chosen entries filled, the others zero */
        G53hExpert chosen[GLM53F_MAX_TOPK + 1];
        memcpy(chosen, tab, (size_t)(K + 1) * sizeof(G53hExpert));
        memset(tab, 0, (size_t)(NE + 1) * sizeof(G53hExpert));
        for (int j = 0; j < K; j++) if (chosen[j].gate.w || chosen[j].gate.flags) tab[ids[j]] = chosen[j];
        tab[NE] = chosen[K];
        if (g53h_h2d_async(tab_d, tab, (size_t)(NE + 1) * sizeof(G53hExpert))) g53_die("glm53f_moe");
        L.n_experts = NE; L.experts = tab_d; L.shared = with_shared ? tab_d + NE : NULL;
        /* FP8 with 128-column blocks: the one-launch decode (which routes again, to the same
         * result); int4 experts and other blocks: the row kernels on the routing already made */
        if (L.block_c == 128 ? g53h_moe(od, xd, 1, &L, NULL, NULL) : g53h_moe_routed_given(od, xd, 1, &L, idx_d, w_d))
            g53_die("glm53f_moe");
    }
    HP(4);
    /* the HBM cache orders each slot's reuse after the kernels launched so far */
    for (int i = 0; i < nh; i++) src->release(src, w->layer, held[i]);
    /* the error flags and the output come back together through the mailbox, one wait */
    const unsigned seq_o = next_seq();
    if (G53_MB_OUT_OFF + 4 * G53H_NERR + ob <= G53H_MBOX_BYTES) {
        if (g53h_publish(G53_MB_OUT, seq_o, G53_MB_OUT_OFF, od, ob)) g53_die("glm53f_moe");
        HP(5);
        if (g53h_mailbox_wait(G53_MB_OUT, seq_o)) g53_die("glm53f_moe");
        HP(6);
        const int *mo = (const int *)((const char *)g53h_mailbox() + G53_MB_OUT_OFF);
        errors_check(mo, w->layer, K);
        if (ob) memcpy(out, mo + G53H_NERR, ob);
    } else {                                         /* a hidden size beyond the mailbox */
        int *errs = (int *)pinned(&g_pin_err, &g_pin_err_n, G53H_NERR * sizeof(int));
        if (g53h_errors_peek_async(errs) || (ob && g53h_d2h_async(out, od, ob)) || g53h_sync()) g53_die("glm53f_moe");
        errors_check(errs, w->layer, K);
    }
}

/* ------------------------------------------------------------- MoE chunk ---- */
/* Host expert views are copied into these per-call staging slots (one per expert in a batch). */
typedef struct { G53Buf b; } G53Slot;
static G53Slot *g_hslots = NULL;
static int g_nhslots = 0;

/* A host view copied into the staging slot at dst + *off, its FP8 codes in the layout the
 * chunk's kernels read (tiled != 0: octet-tiled, for a tiled grouped pass; else row-major). */
static G53hMat stage_mat(const Glm53fMat *m, uint8_t *dst, size_t *off, int tiled)
{
    G53hMat d;
    memset(&d, 0, sizeof d);
    const size_t cb = mat_code_bytes(m), sb = mat_scale_bytes(m);
    uint8_t *w = dst + *off;
    *off += (cb + 255) & ~(size_t)255;
    uint8_t *s = dst + *off;
    *off += (sb + 255) & ~(size_t)255;
    const int is_t = m->dt == GLM53F_WF8T;
    int steps_done = 0;
    if (m->dt == GLM53F_WI4T) {                                /* int4 levels back to rows */
        uint8_t *t = (uint8_t *)buf_get(&g_tile_stage, cb);
        if (g53h_h2d(t, m->w, cb) || g53h_tile_i4(w, t, m->rows, m->cols, 1)) g53_die("copying a host expert to HBM");
    } else if (m->dt == GLM53F_WI4M) {                         /* levels and steps back to rows */
        uint8_t *t = (uint8_t *)buf_get(&g_tile_stage, ((cb + 255) & ~(size_t)255) + sb);
        float *ts = (float *)(t + ((cb + 255) & ~(size_t)255));
        if (g53h_h2d(t, m->w, cb) || g53h_h2d(ts, m->s, sb) ||
            g53h_mtile_i4(w, (float *)s, t, ts, m->rows, m->cols, 1))
            g53_die("copying a host expert to HBM");
        steps_done = 1;
    } else if (m->dt == GLM53F_WF8M) {        /* MFMA-tiled: back to rows, octet-tiled if asked */
        uint8_t *t = (uint8_t *)buf_get(&g_tile_stage, 2 * cb);
        if (g53h_h2d(t, m->w, cb) ||
            (tiled ? (g53h_mtile_f8(t + cb, t, m->rows, m->cols, 1) || g53h_tile_f8(w, t + cb, m->rows, m->cols))
                   : g53h_mtile_f8(w, t, m->rows, m->cols, 1)))
            g53_die("copying a host expert to HBM");
    } else if (m->dt != GLM53F_WI4 && is_t != (tiled != 0)) {  /* convert on the way in */
        uint8_t *t = (uint8_t *)buf_get(&g_tile_stage, cb);
        if (g53h_h2d(t, m->w, cb) ||
            (is_t ? g53h_untile_f8(w, t, m->rows, m->cols) : g53h_tile_f8(w, t, m->rows, m->cols)))
            g53_die("copying a host expert to HBM");
    } else if (g53h_h2d(w, m->w, cb)) {
        g53_die("copying a host expert to HBM");
    }
    if (!steps_done && g53h_h2d(s, m->s, sb)) g53_die("copying a host expert to HBM");
    d.w = w; d.s = (const float *)s;
    d.rows = m->rows; d.cols = m->cols; d.br = m->br; d.bc = m->bc; d.scols = m->scols;
    d.flags = mat_i4(m) ? G53H_MAT_I4 : (tiled ? G53H_MAT_TILED : 0);
    return d;
}

/* Staging bytes of one expert's three matrices (stage_mat / chunk_view pad each part to 256). */
static size_t expert_stage_bytes(const Glm53fExpertQ *q)
{
    const Glm53fMat *ms[3] = {&q->gate, &q->up, &q->down};
    size_t n = 0;
    for (int i = 0; i < 3; i++)
        n += ((mat_code_bytes(ms[i]) + 255) & ~(size_t)255) + ((mat_scale_bytes(ms[i]) + 255) & ~(size_t)255);
    return n;
}

/* An HBM view as the chunk's kernels read it: in place when its FP8 layout is the one they read
 * (tiled != 0: octet-tiled, else row-major), otherwise converted into the staging slot (ordered
 * on the stream before the kernels that read it). Int4 views are used as they are, except
 * int4-tiled ones, whose levels are untiled into the staging slot (the steps are read in place). */
static G53hMat chunk_view(const Glm53fMat *m, uint8_t *dst, size_t *off, int tiled)
{
    G53hMat d = view_mat_f8(m);
    if (m->dt == GLM53F_WI4M) {                   /* levels and steps untiled into the slot */
        uint8_t *w = dst + *off;
        *off += (mat_code_bytes(m) + 255) & ~(size_t)255;
        float *st = (float *)(dst + *off);
        *off += (mat_scale_bytes(m) + 255) & ~(size_t)255;
        if (g53h_mtile_i4(w, st, (const uint8_t *)m->w, m->s, m->rows, m->cols, 1))
            g53_die("converting an int4 expert view");
        d.w = w; d.s = st;
        d.flags = G53H_MAT_I4;
        return d;
    }
    if (m->dt == GLM53F_WI4T) {
        uint8_t *w = dst + *off;
        *off += (mat_code_bytes(m) + 255) & ~(size_t)255;
        if (g53h_tile_i4(w, (const uint8_t *)m->w, m->rows, m->cols, 1)) g53_die("converting an int4 expert view");
        d.w = w;
        d.flags = G53H_MAT_I4;
        return d;
    }
    if (m->dt == GLM53F_WF8M) {                   /* MFMA-tiled: back to rows, octet-tiled if asked */
        uint8_t *w = dst + *off;
        const size_t cb = mat_code_bytes(m);
        *off += (cb + 255) & ~(size_t)255;
        uint8_t *t = tiled ? (uint8_t *)buf_get(&g_tile_stage, cb) : w;
        if (g53h_mtile_f8(t, (const uint8_t *)m->w, m->rows, m->cols, 1) ||
            (tiled && g53h_tile_f8(w, t, m->rows, m->cols)))
            g53_die("converting an expert view");
        d.w = w;
        d.flags = tiled ? G53H_MAT_TILED : 0;
        return d;
    }
    const int is_t = m->dt == GLM53F_WF8T;
    if (m->dt == GLM53F_WI4 || is_t == (tiled != 0)) return d;
    uint8_t *w = dst + *off;
    *off += (mat_code_bytes(m) + 255) & ~(size_t)255;
    if (is_t ? g53h_untile_f8(w, (const uint8_t *)m->w, m->rows, m->cols)
             : g53h_tile_f8(w, (const uint8_t *)m->w, m->rows, m->cols))
        g53_die("converting an expert view");
    d.w = w;
    d.flags = tiled ? G53H_MAT_TILED : 0;
    return d;
}

#define G53_MOE_BATCH 16                /* reference's getmany batch (src/core/glm53f_ops.c:989) */

/* One chunk of T <= 64 tokens (reference moe_chunk, src/core/glm53f_ops.c:1144-1342). */
static void moe_chunk(float *out, const float *x, const Glm53fMoeW *w, const Glm53fCfg *c, int T, int with_shared)
{
    const int E = c->hidden, K = c->topk, NE = c->n_experts;
    Glm53fExpertSrc *src = w->src;
    if (T == 1 && g53h_cache_is(src)) {
        decode_cached(out, x, w, c, with_shared);
        return;
    }
    const float *xd = stage_in(&g_xin, x, (size_t)T * E);
    int *idx_d = (int *)buf_get(&g_idx, ((size_t)T * K + 1) * sizeof(int));
    float *w_d = (float *)buf_get(&g_w, (size_t)T * K * sizeof(float));
    /* routing of every token, read back with the NaN flag in one copy */
    {
        int dt = 0;
        const void *gate = resident_router(w->gate, (size_t)NE * E, &dt);
        const float *bias = (const float *)resident(w->bias, (size_t)NE * sizeof(float));
        int *flag_d = idx_d + (size_t)T * K;
        if (g53h_memset(flag_d, 0, sizeof(int)) ||
            g53h_router(idx_d, w_d, xd, T, gate, dt, bias, NE, E, K, c->norm_topk, c->routed_scale, flag_d))
            g53_die("glm53f_router");
    }
    int *ids = (int *)pinned(&g_pin_back, &g_pin_back_n, ((size_t)64 * GLM53F_MAX_TOPK + 1 + 1024) * sizeof(int));
    if (g53h_d2h(ids, idx_d, ((size_t)T * K + 1) * sizeof(int))) g53_die("glm53f_moe routing");
    if (ids[(size_t)T * K]) {
        fprintf(stderr, "glm53f: FATAL, router selection (NaN scores) is below %d, above the limit of %d.\n", K, K);
        abort();
    }
    int uniq[64 * GLM53F_MAX_TOPK], nu = 0;
    unsigned char seen[1024];
    memset(seen, 0, (size_t)NE);
    for (int i = 0; i < T * K; i++)
        if (!seen[ids[i]]) { seen[ids[i]] = 1; uniq[nu++] = ids[i]; }
    if (T == 1) route_top16(w->layer, xd, w, c);

    read_switches();
    const int prefetch = w->prefetch_n > 0 && src->hint != NULL && (T == 1 || !g_prefill_off);
    if (prefetch) {
        src->hint(src, w->layer, uniq, nu);
        if (w->next_gate) {
            int per = (T > 1 && g_prefill_pred >= 0) ? g_prefill_pred : w->prefetch_n;
            if (per > 2 * GLM53F_MAX_TOPK) per = 2 * GLM53F_MAX_TOPK;
            if (per > NE) per = NE;
            static int pred[64 * 2 * GLM53F_MAX_TOPK];
            if (T == 1) {
                const int np = per > 0 ? predict_next(pred, xd, w, c, 1, per) : 0;
                src->hint(src, w->layer + 1, pred, np);
            } else if (per > 0 && (w->prefill_next || g_prefill_pred >= 0)) {
                const int np = predict_next(pred, xd, w, c, T, per);
                src->hint(src, w->layer + 1, pred, np);
            }
        }
    }

    /* the unique experts in first-seen order, in the reference's getmany batches of 16; within a
     * batch at most topk of them are held at once (a cache of topk + 1 slots, the reference's
     * minimum, must always find a victim), multiplied together and then released.
     * Contributions are kept per (token, slot) and combined in top-k order at the end, so the
     * batching does not change the result. */
    const int B = K < G53_MOE_BATCH ? K : G53_MOE_BATCH;
    if (g_nhslots < B) {
        G53Slot *ns = (G53Slot *)realloc(g_hslots, (size_t)B * sizeof *ns);
        if (!ns) { fprintf(stderr, "glm53f: FATAL, out of host memory\n"); abort(); }
        memset(ns + g_nhslots, 0, (size_t)(B - g_nhslots) * sizeof *ns);
        g_hslots = ns;
        g_nhslots = B;
    }
    const int nslots = K + (with_shared ? 1 : 0);
    G53hExpert *table_d = (G53hExpert *)buf_get(&g_table, (size_t)(NE + 1) * sizeof(G53hExpert));
    G53hExpert *table = (G53hExpert *)pinned(&g_pin_tab, &g_pin_tab_n, (size_t)(NE + 1) * sizeof(G53hExpert));
    G53hMoeLayer L;
    memset(&L, 0, sizeof L);
    L.hidden = E; L.inter = c->moe_inter; L.n_experts = NE; L.topk = K; L.norm_topk = c->norm_topk;
    L.routed_scale = c->routed_scale; L.swiglu_limit = c->swiglu_limit;
    L.experts = table_d;
    L.block_c = 128;
    /* a chunk of tokens takes the grouped matrix-core kernels when the layer qualifies: every
     * batch of fetched experts is multiplied for all its tokens at once. The experts' format is
     * known once the first batch is fetched: FP8 with 128-column blocks takes the grouped path,
     * anything else (int4 experts, other blocks) the exact row kernels. */
    int grouped = T >= 2 && T <= g53h_grouped_max_tokens(&L) &&
                  (!with_shared || (w->sh_gate.dt == GLM53F_WF8 && w->sh_up.dt == GLM53F_WF8 &&
                                    w->sh_down.dt == GLM53F_WF8 && w->sh_gate.bc == 128 && w->sh_up.bc == 128 &&
                                    w->sh_down.bc == 128)) ? -1 : 0;
    float *contrib = NULL;
    int held[GLM53F_MAX_TOPK];
    int first = 1;
    /* the FP8 layout the chunk's kernels read: octet-tiled when a grouped pass is possible and
     * the first expert view is tiled (the HBM cache's slots: used in place) and the shared
     * expert can be kept tiled; row-major otherwise. Views of the other layout are converted. */
    int want_tiled = grouped ? -1 : 0;
    for (int g0 = 0; g0 < nu || (g0 == 0 && with_shared); g0 += G53_MOE_BATCH) {
        const int gn = (nu - g0) < G53_MOE_BATCH ? (nu - g0) : G53_MOE_BATCH;
        if (gn > 0 && !prefetch && src->getmany) src->getmany(src, w->layer, uniq + g0, gn);
        for (int b0 = g0; b0 < g0 + gn || (first && with_shared); b0 += B) {
            const int bn = (g0 + gn - b0) < B ? (g0 + gn - b0) : B;
            int nh = 0, block_c = 128, any_i4 = 0;
            memset(table, 0, (size_t)NE * sizeof(G53hExpert));
            for (int u = b0; u < b0 + bn; u++) {
                const int e = uniq[u];
                Glm53fExpertQ q;
                memset(&q, 0, sizeof q);
                if (src->get(src, w->layer, e, &q) != 0) {
                    glm53f_expert_drops++;
                    fprintf(stderr, "EXPERT DROP: layer %d expert %d failed to load; this output is CORRUPT\n",
                            w->layer, e);
                    table[e].gate.flags = G53H_MAT_DROPPED;   /* its contributions are zero */
                    continue;
                }
                check_expert_shape(&q, c, w->layer, e);
                const int q_i4 = mat_i4(&q.gate) || mat_i4(&q.up) || mat_i4(&q.down);
                if (q_i4) any_i4 = 1;
                if (q.gate.bc != 128 || q.up.bc != 128 || q.down.bc != 128 || any_i4) block_c = 0;
                if (want_tiled < 0)
                    want_tiled = q.gate.dt == GLM53F_WF8T && q.up.dt == GLM53F_WF8T && q.down.dt == GLM53F_WF8T &&
                                 (!with_shared || shared_tileable(w));
                if (want_tiled == 1 && block_c != 128) {
                    fprintf(stderr, "glm53f: FATAL, layer %d mixes octet-tiled FP8 experts with other formats in one "
                                    "chunk\n", w->layer);
                    abort();
                }
                const int tl = want_tiled == 1;
                const size_t need = expert_stage_bytes(&q);
                const int dev = g53h_is_device_ptr(q.gate.w);
                size_t off = 0;
                if (dev) {
                    /* FP8 views in the other layout, and int4-tiled views (their levels are
                     * untiled), are converted into the staging slot */
                    const int conv = (!mat_i4(&q.gate) && (q.gate.dt == GLM53F_WF8T) != tl) ||
                                     (!mat_i4(&q.up) && (q.up.dt == GLM53F_WF8T) != tl) ||
                                     (!mat_i4(&q.down) && (q.down.dt == GLM53F_WF8T) != tl) ||
                                     q.gate.dt == GLM53F_WI4T || q.up.dt == GLM53F_WI4T || q.down.dt == GLM53F_WI4T ||
                                     q.gate.dt == GLM53F_WI4M || q.up.dt == GLM53F_WI4M || q.down.dt == GLM53F_WI4M ||
                                     q.gate.dt == GLM53F_WF8M || q.up.dt == GLM53F_WF8M || q.down.dt == GLM53F_WF8M;
                    uint8_t *dst = conv ? (uint8_t *)buf_get(&g_hslots[u - b0].b, need) : NULL;
                    held[nh++] = e;                      /* released once its kernels are queued */
                    table[e].gate = chunk_view(&q.gate, dst, &off, tl);
                    table[e].up = chunk_view(&q.up, dst, &off, tl);
                    table[e].down = chunk_view(&q.down, dst, &off, tl);
                } else {
                    uint8_t *dst = (uint8_t *)buf_get(&g_hslots[u - b0].b, need);
                    table[e].gate = stage_mat(&q.gate, dst, &off, tl);
                    table[e].up = stage_mat(&q.up, dst, &off, tl);
                    table[e].down = stage_mat(&q.down, dst, &off, tl);
                    /* the copies have completed: hand the views back at once, in the reference's
                     * get / release order (src/core/glm53f_ops.c:1256-1328) */
                    if (src->release) src->release(src, w->layer, e);
                }
            }
            L.shared = NULL;
            if (with_shared && first) {              /* the shared expert rides with the first batch */
                G53hExpert sh;
                if (want_tiled < 0) want_tiled = 0;   /* no routed view in the first batch */
                if ((any_i4 || want_tiled == 1) && shared_tileable(w)) {  /* tiled kernels, or the row-wave fast path */
                    sh.gate = dev_mat_resident_tiled(&w->sh_gate, "shared gate");
                    sh.up = dev_mat_resident_tiled(&w->sh_up, "shared up");
                    sh.down = dev_mat_resident_tiled(&w->sh_down, "shared down");
                } else {
                    sh.gate = dev_mat_resident(&w->sh_gate, "shared gate");
                    sh.up = dev_mat_resident(&w->sh_up, "shared up");
                    sh.down = dev_mat_resident(&w->sh_down, "shared down");
                }
                if (w->sh_gate.bc != 128 || w->sh_up.bc != 128 || w->sh_down.bc != 128 ||
                    (sh.gate.flags && want_tiled != 1))
                    block_c = 0;
                table[NE] = sh;
                if (g53h_h2d_async(table_d + NE, table + NE, sizeof sh)) g53_die("glm53f_moe");
                L.shared = table_d + NE;
            }
            if (g53h_h2d_async(table_d, table, (size_t)NE * sizeof(G53hExpert))) g53_die("glm53f_moe");
            L.block_c = block_c;
            if (grouped < 0) {                       /* decided by the first batch */
                int present = 0;
                for (int u = b0; u < b0 + bn; u++) if (table[uniq[u]].gate.w) present = 1;
                grouped = block_c == 128 && present;
                if (want_tiled == 1 && !grouped) {
                    fprintf(stderr, "glm53f: FATAL, layer %d: octet-tiled experts without a grouped pass\n", w->layer);
                    abort();
                }
                L.tiled = grouped && want_tiled == 1;
                if (!grouped) want_tiled = 0;        /* the exact kernels read row-major codes */
                if (grouped) {                       /* the plan reserves the shared expert's rows */
                    const G53hExpert *keep_shared = L.shared;
                    L.shared = with_shared ? table_d + NE : NULL;
                    if (g53h_grouped_begin(xd, T, &L, idx_d)) g53_die("glm53f_moe");
                    L.shared = keep_shared;
                }
            }
            if (!grouped && !contrib) contrib = (float *)buf_get(&g_contrib, (size_t)T * nslots * E * sizeof(float));
            if (grouped) {
                if (block_c != 128) {
                    fprintf(stderr, "glm53f: FATAL, a routed expert of layer %d has no 128-column blocks\n", w->layer);
                    abort();
                }
                if (g53h_grouped_batch(&L)) g53_die("glm53f_moe");
            } else if (L.shared) {
                if (g53h_moe_partial(contrib, xd, T, &L, idx_d)) g53_die("glm53f_moe");
            } else {
                /* a layout with the shared slot still has K+1 slots per token */
                if (with_shared) {
                    G53hExpert none;
                    memset(&none, 0, sizeof none);
                    table[NE] = none;
                    if (g53h_h2d_async(table_d + NE, table + NE, sizeof none)) g53_die("glm53f_moe");
                    L.shared = table_d + NE;
                }
                if (g53h_moe_partial(contrib, xd, T, &L, idx_d)) g53_die("glm53f_moe");
            }
            first = 0;
            /* release the batch once the kernels that read it are done: the HBM cache orders that
             * on the device (release records an event its next copy into the slot waits for); any
             * other source, and the pinned table rewritten for the next batch, wait for the stream */
            if (g53h_sync()) g53_die("glm53f_moe");
            if (src->release)
                for (int i = 0; i < nh; i++) src->release(src, w->layer, held[i]);
            if (bn <= 0) break;
        }
    }
    L.shared = with_shared ? table_d + NE : NULL;
    const int odev = g53h_is_device_ptr(out);
    float *od = odev ? out : (float *)buf_get(&g_out, (size_t)T * E * sizeof(float));
    if (grouped) {
        if (g53h_grouped_end(od, w_d)) g53_die("glm53f_moe");
    } else if (g53h_moe_combine(od, contrib, w_d, T, &L)) {
        g53_die("glm53f_moe");
    }
    int *errs = errors_enqueue();
    if (!odev) {
        if (g53h_d2h(out, od, (size_t)T * E * sizeof(float))) g53_die("glm53f_moe");
    } else if (g53h_sync()) {
        g53_die("glm53f_moe");
    }
    errors_check(errs, w->layer, K);
}

static void moe_layer(float *out, const float *x, const Glm53fMoeW *w, const Glm53fCfg *c, int T, int with_shared)
{
    if (T < 1) return;
    ensure_device();
    if (c->n_experts > 1024) {
        fprintf(stderr, "glm53f: FATAL, routed experts is %d, above the limit of 1024.\n", c->n_experts);
        abort();
    }
    /* chunks of 64 tokens, as src/core/glm53f_ops.c:1344-1362 */
    for (int t0 = 0; t0 < T; t0 += G53_MOE_CHUNK) {
        const int n = (T - t0) < G53_MOE_CHUNK ? (T - t0) : G53_MOE_CHUNK;
        moe_chunk(out + (size_t)t0 * c->hidden, x + (size_t)t0 * c->hidden, w, c, n, with_shared);
    }
}

void glm53f_moe(float *out, const float *x, const Glm53fMoeW *w, const Glm53fCfg *c, int T,
                float *scratch)
{
    (void)scratch;
    moe_layer(out, x, w, c, T, 1);
}

void glm53f_moe_routed(float *out, const float *x, const Glm53fMoeW *w, const Glm53fCfg *c, int T,
                       float *scratch)
{
    (void)scratch;
    moe_layer(out, x, w, c, T, 0);
}
