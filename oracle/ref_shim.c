/* ref_shim.c - a flat C entry layer over the reference's own expert path, for the tests.
 *
 * TEST INFRASTRUCTURE ONLY. Compiled together with the reference's unmodified sources
 * (src/core/glm53f_ops.c, src/core/glm53f_dsa.c, read where they lie under /root/reference)
 * into oracle/_ref/libglm53f_ref.so by oracle/Makefile. The reference's header types are
 * used as the reference declares them. Experts are served from caller memory through an
 * in-memory Glm53fExpertSrc (get returns views, release does nothing; a NULL gate marks a
 * failed load), which is the seam the reference's own docs name for faking the source.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "glm53f.h"

typedef struct {
    const uint8_t *gw, *uw, *dw;
    const float   *gs, *us, *ds;
} RefExpert;

typedef struct {
    Glm53fExpertSrc src;              /* first member: the MoE passes &src back */
    const RefExpert *ex;
    int E, I, br, bc;
    int i4;                           /* routed experts are GLM53F_WI4 (q, steps) */
} MemSrc;

static void fill(Glm53fMat *m, const uint8_t *w, const float *s, int rows, int cols, int br, int bc)
{
    memset(m, 0, sizeof *m);
    m->w = w; m->s = s; m->dt = GLM53F_WF8;
    m->rows = rows; m->cols = cols; m->br = br; m->bc = bc; m->scols = (cols + bc - 1) / bc;
}

static void fill_i4(Glm53fMat *m, const uint8_t *q, const float *steps, int rows, int cols)
{
    memset(m, 0, sizeof *m);
    m->w = q; m->s = steps; m->dt = GLM53F_WI4;
    m->rows = rows; m->cols = cols; m->br = 1; m->bc = GLM53F_I4_GROUP; m->scols = cols / GLM53F_I4_GROUP;
}

static int mem_get(Glm53fExpertSrc *self, int layer, int e, Glm53fExpertQ *q)
{
    (void)layer;
    MemSrc *m = (MemSrc *)self;
    const RefExpert *x = &m->ex[e];
    if (!x->gw) return -1;
    if (m->i4) {
        fill_i4(&q->gate, x->gw, x->gs, m->I, m->E);
        fill_i4(&q->up, x->uw, x->us, m->I, m->E);
        fill_i4(&q->down, x->dw, x->ds, m->E, m->I);
        return 0;
    }
    fill(&q->gate, x->gw, x->gs, m->I, m->E, m->br, m->bc);
    fill(&q->up, x->uw, x->us, m->I, m->E, m->br, m->bc);
    fill(&q->down, x->dw, x->ds, m->E, m->I, m->br, m->bc);
    return 0;
}

static void cfg_of(Glm53fCfg *c, int E, int I, int NE, int K, int br, int bc, int norm_topk,
                   float routed_scale, float limit)
{
    memset(c, 0, sizeof *c);
    c->hidden = E; c->moe_inter = I; c->n_experts = NE; c->topk = K; c->n_shared = 1;
    c->routed_scale = routed_scale; c->norm_topk = norm_topk; c->swiglu_limit = limit;
    c->fp8_block_r = br; c->fp8_block_c = bc; c->n_layers = 1;
}

static long moe_any(float *out, const float *x, int T, int E, int I, int NE, int K, int br, int bc,
                    int norm_topk, float routed_scale, float limit, const float *gate, const float *bias,
                    const RefExpert *experts, const RefExpert *shared, int i4);

long ref_moe(float *out, const float *x, int T, int E, int I, int NE, int K, int br, int bc,
             int norm_topk, float routed_scale, float limit, const float *gate, const float *bias,
             const RefExpert *experts, const RefExpert *shared)
{
    return moe_any(out, x, T, E, I, NE, K, br, bc, norm_topk, routed_scale, limit, gate, bias, experts, shared, 0);
}

/* The same with GLM53F_WI4 routed experts ({q, steps} per matrix, as glm53f_i4_from_f8 writes
 * them) and the FP8 shared expert: the reference's --experts int4 mode. */
long ref_moe_i4(float *out, const float *x, int T, int E, int I, int NE, int K, int br, int bc,
                int norm_topk, float routed_scale, float limit, const float *gate, const float *bias,
                const RefExpert *experts, const RefExpert *shared)
{
    return moe_any(out, x, T, E, I, NE, K, br, bc, norm_topk, routed_scale, limit, gate, bias, experts, shared, 1);
}

/* glm53f_i4_from_f8 on an FP8 matrix; glm53f_mm_batch on a GLM53F_WI4 one. */
void ref_i4_from_f8(uint8_t *q, float *steps, const uint8_t *W, const float *S, int rows, int cols, int br, int bc)
{
    Glm53fMat m;
    fill(&m, W, S, rows, cols, br, bc);
    glm53f_i4_from_f8(q, steps, &m);
}

void ref_mm_i4(float *y, const float *x, int T, const uint8_t *q, const float *steps, int rows, int cols)
{
    Glm53fMat m;
    fill_i4(&m, q, steps, rows, cols);
    if (T == 1) glm53f_mm(y, x, &m);
    else glm53f_mm_batch(y, x, T, &m);
}

static long moe_any(float *out, const float *x, int T, int E, int I, int NE, int K, int br, int bc,
                    int norm_topk, float routed_scale, float limit, const float *gate, const float *bias,
                    const RefExpert *experts, const RefExpert *shared, int i4)
{
    Glm53fCfg c;
    cfg_of(&c, E, I, NE, K, br, bc, norm_topk, routed_scale, limit);
    MemSrc src;
    memset(&src, 0, sizeof src);
    src.src.get = mem_get;
    src.src.ctx = &src;
    src.ex = experts; src.E = E; src.I = I; src.br = br; src.bc = bc; src.i4 = i4;
    Glm53fMoeW w;
    memset(&w, 0, sizeof w);
    w.gate = gate; w.bias = bias; w.src = &src.src; w.layer = 0;
    if (shared) {
        fill(&w.sh_gate, shared->gw, shared->gs, I, E, br, bc);
        fill(&w.sh_up, shared->uw, shared->us, I, E, br, bc);
        fill(&w.sh_down, shared->dw, shared->ds, E, I, br, bc);
    }
    float *scratch = (float *)malloc(glm53f_moe_scratch(&c, T) * sizeof(float));
    if (!scratch) return -1;
    const long drops0 = glm53f_expert_drops;
    if (shared) glm53f_moe(out, x, &w, &c, T, scratch);
    else glm53f_moe_routed(out, x, &w, &c, T, scratch);
    free(scratch);
    return glm53f_expert_drops - drops0;
}

void ref_router(int *idx, float *wt, const float *x, int E, int NE, int K, int norm_topk,
                float routed_scale, const float *gate, const float *bias)
{
    Glm53fCfg c;
    cfg_of(&c, E, 1, NE, K, 128, 128, norm_topk, routed_scale, 10.0f);
    Glm53fMoeW w;
    memset(&w, 0, sizeof w);
    w.gate = gate; w.bias = bias;
    glm53f_router(idx, wt, x, &w, &c);
}

void ref_mm(float *y, const float *x, int T, const uint8_t *W, const float *S, int rows, int cols,
            int br, int bc)
{
    Glm53fMat m;
    fill(&m, W, S, rows, cols, br, bc);
    if (T == 1) glm53f_mm(y, x, &m);
    else glm53f_mm_batch(y, x, T, &m);
}

void ref_swiglu(float *y, const float *gu, int n, float limit) { glm53f_swiglu_clamp(y, gu, n, limit); }

float ref_e4m3f(uint8_t b) { return glm53f_e4m3f(b); }

/* The reference's expert-source protocol, recorded: the same in-memory experts behind a source
 * whose get / release / getmany / hint append to a log ([1, layer, e] get, [2, layer, e]
 * release, [3, layer, n, ids...] getmany, [4, layer, n, ids...] hint), with the next layer's
 * router for the prediction. Returns the log length (ints), or -1 when it would overflow. */
typedef struct {
    MemSrc m;
    int *log, cap, n, bad;
} LogSrc;

static void logv(LogSrc *s, int v)
{
    if (s->n < s->cap) s->log[s->n++] = v;
    else s->bad = 1;
}

static int log_get(Glm53fExpertSrc *self, int layer, int e, Glm53fExpertQ *q)
{
    LogSrc *s = (LogSrc *)self;
    logv(s, 1); logv(s, layer); logv(s, e);
    return mem_get(self, layer, e, q);
}

static void log_release(Glm53fExpertSrc *self, int layer, int e)
{
    LogSrc *s = (LogSrc *)self;
    logv(s, 2); logv(s, layer); logv(s, e);
}

static int log_getmany(Glm53fExpertSrc *self, int layer, const int *ids, int n)
{
    LogSrc *s = (LogSrc *)self;
    logv(s, 3); logv(s, layer); logv(s, n);
    for (int i = 0; i < n; i++) logv(s, ids[i]);
    return 0;
}

static void log_hint(Glm53fExpertSrc *self, int layer, const int *ids, int n)
{
    LogSrc *s = (LogSrc *)self;
    logv(s, 4); logv(s, layer); logv(s, n);
    for (int i = 0; i < n; i++) logv(s, ids[i]);
}

int ref_moe_proto(float *out, const float *x, int T, int E, int I, int NE, int K, int br, int bc,
                  int norm_topk, float routed_scale, float limit, const float *gate, const float *bias,
                  const RefExpert *experts, const RefExpert *shared, int layer, const float *next_gate,
                  const float *next_bias, int prefetch_n, int prefill_next, int with_hint, int with_getmany,
                  int *log, int cap)
{
    Glm53fCfg c;
    cfg_of(&c, E, I, NE, K, br, bc, norm_topk, routed_scale, limit);
    c.n_layers = layer + 2;
    LogSrc src;
    memset(&src, 0, sizeof src);
    src.m.src.get = log_get;
    src.m.src.release = log_release;
    src.m.src.getmany = with_getmany ? log_getmany : NULL;
    src.m.src.hint = with_hint ? log_hint : NULL;
    src.m.src.ctx = &src;
    src.m.ex = experts; src.m.E = E; src.m.I = I; src.m.br = br; src.m.bc = bc;
    src.log = log; src.cap = cap;
    Glm53fMoeW w;
    memset(&w, 0, sizeof w);
    w.gate = gate; w.bias = bias; w.src = &src.m.src; w.layer = layer;
    w.next_gate = next_gate; w.next_bias = next_bias;
    w.prefetch_n = prefetch_n; w.prefill_next = prefill_next;
    if (shared) {
        fill(&w.sh_gate, shared->gw, shared->gs, I, E, br, bc);
        fill(&w.sh_up, shared->uw, shared->us, I, E, br, bc);
        fill(&w.sh_down, shared->dw, shared->ds, E, I, br, bc);
    }
    float *scratch = (float *)malloc(glm53f_moe_scratch(&c, T) * sizeof(float));
    if (!scratch) return -1;
    glm53f_moe(out, x, &w, &c, T, scratch);
    free(scratch);
    return src.bad ? -1 : src.n;
}
