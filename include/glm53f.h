/* glm53f.h - the routed-expert MoE boundary of the GLM-5.3-Flash engine, served by MI355X.
 *
 * This header is the drop-in surface: the same types, field order and function signatures
 * as the reference engine's public header, restricted to the expert path, so host code that
 * was compiled against the reference keeps compiling and keeps its struct layouts. Behind
 * these symbols every product runs on one gfx950 GPU (hand-written HIP kernels, see g53h.h);
 * there is no CPU arithmetic path in this library.
 *
 * Reference interface replaced (file:line in josesilva05/glm-5.3-flash-in-c):
 *   Glm53fCfg                 include/glm53f/glm53f.h:47-95
 *   Glm53fMat, GLM53F_W*      include/glm53f/glm53f.h:121-134
 *   glm53f_mm / _mm_batch     include/glm53f/glm53f.h:136-142  (src/core/glm53f_ops.c:185-228, 376-458)
 *   glm53f_e4m3f, bf16f       include/glm53f/glm53f.h:149-159  (src/core/glm53f_ops.c:48-72)
 *   glm53f_swiglu_clamp       include/glm53f/glm53f.h:167      (src/core/glm53f_ops.c:486-494)
 *   Glm53fExpertQ/ExpertSrc   include/glm53f/glm53f.h:211-228
 *   Glm53fMoeW                include/glm53f/glm53f.h:230-247
 *   glm53f_router             include/glm53f/glm53f.h:339      (src/core/glm53f_ops.c:945-976)
 *   glm53f_moe(_routed,_scratch) include/glm53f/glm53f.h:341-349 (src/core/glm53f_ops.c:988-1000, 1144-1362)
 *   glm53f_mlp(_scratch)      include/glm53f/glm53f.h:351-353  (src/core/glm53f_ops.c:496-511)
 *   glm53f_expert_drops, glm53f_quiet   include/glm53f/glm53f.h:288-295
 *
 * POINTERS. Every pointer argument may be host memory (as the reference takes it) or HBM
 * (device memory of the current g53h device). Host operands are staged to HBM; weights given
 * as host pointers are uploaded once and kept resident, keyed by their host address, so the
 * caller must not change the bytes behind a host weight pointer after first use (call
 * glm53f_forget_host_weights() if it does). Expert views returned by an Glm53fExpertSrc may
 * likewise be host or device; the HBM expert cache (glm53f_cache.h) returns device views.
 *
 * ERRORS follow the reference: a HIP failure inside a void kernel prints and aborts, a routed
 * expert whose get() fails is counted in glm53f_expert_drops and its contribution is zero,
 * NaN routing aborts.
 */
#ifndef GLM53F_H
#define GLM53F_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GLM53F_MAX_LAYERS 256
#define GLM53F_MAX_TOPK   64
#define GLM53F_MAX_HC     8
#define GLM53F_MAX_EOS    8

/* Model configuration. Field order and types are the reference's, so a caller's struct is
 * read as written; the expert path reads hidden, n_experts, topk, n_shared, moe_inter,
 * routed_scale, norm_topk, swiglu_limit and fp8_block_r/c. The rest is carried for layout. */
typedef struct {
    int   hidden;
    int   n_layers;
    int   vocab;
    float rms_eps;

    int   hc_mult;
    int   hc_iters;
    float hc_eps;

    int   kda_heads;
    int   kda_head_dim;
    int   conv_k;
    float gate_lb;

    int   n_heads;
    int   q_lora;
    int   kv_lora;
    int   qk_nope;
    int   v_head;
    int   index_topk;
    int   index_kpool;
    int   index_heads;
    int   index_dim;
    int   index_tail;

    int   n_experts;         /* routed experts per MoE layer (288)          */
    int   topk;              /* experts per token (8)                        */
    int   n_shared;          /* shared experts (1)                           */
    int   moe_inter;         /* expert intermediate size (2048)              */
    int   dense_inter;
    float routed_scale;      /* routed weights are multiplied by this (2.5)  */
    int   norm_topk;         /* renormalise the top-k weights to sum to one  */
    float swiglu_limit;      /* SwiGLU clamp (10)                            */

    int   fp8_block_r, fp8_block_c;   /* FP8 scale block (128 x 128)           */

    unsigned char is_mla[GLM53F_MAX_LAYERS];
    unsigned char is_dense[GLM53F_MAX_LAYERS];

    int   eos[GLM53F_MAX_EOS];
    int   n_eos;
} Glm53fCfg;

/* Storage formats of a matrix. GLM53F_WF8 and GLM53F_WI4 are multiplied on the GPU by this
 * library; the router is fp32 (GLM53F_WF32) or bf16 (GLM53F_WBF16) bit patterns. GLM53F_WF8T is this
 * library's own: the expert views of its HBM cache (glm53f_cache.h) hold the same E4M3 codes in
 * the octet-tiled layout of g53h.h (G53H_MAT_TILED), for its kernels; the reference never makes
 * one. GLM53F_WI4T, also this library's own: the int4 views of its cache in int4 mode 2 (the
 * levels int4-tiled, G53H_MAT_I4T of g53h.h; the steps as GLM53F_WI4's). GLM53F_WI4M, also
 * this library's own: the int4 views of its cache in int4 mode 3 (levels and steps int4
 * MFMA-tiled, G53H_MAT_I4 | G53H_MAT_MTILED of g53h.h, the layout of the FP4 matrix-core decode).
 * GLM53F_WF8M, also this library's own: the FP8 views of its cache with GLM53F_CACHE_MFMA set
 * (E4M3 codes MFMA-tiled, G53H_MAT_MTILED, the layout of the FP8 matrix-core decode). */
enum { GLM53F_WF32 = 0, GLM53F_WBF16 = 1, GLM53F_WF8 = 2, GLM53F_WI4 = 3, GLM53F_WF8T = 0x102, GLM53F_WI4T = 0x103,
       GLM53F_WI4M = 0x104, GLM53F_WF8M = 0x105 };

/* Group size of the GLM53F_WI4 matrices the reference's engine produces
 * (include/glm53f/glm53f.h:124-125). */
#define GLM53F_I4_GROUP 64

/* A self-describing matrix. For GLM53F_WF8, w holds rows*cols E4M3 codes row-major and s
 * the fp32 block scales [ceil(rows/br)][scols]; element (i,j) = E4M3(w[i*cols+j]) *
 * s[(i/br)*scols + j/bc]. For GLM53F_WI4 (include/glm53f/glm53f.h:115-121), w holds
 * rows*cols/2 bytes of signed 4-bit levels, two per byte (the even column in the low nibble,
 * level = nibble - 8), and s one fp32 step per row and group of bc columns [rows][scols];
 * element (i,j) = level(i,j) * s[i*scols + j/bc]. */
typedef struct {
    const void  *w;
    const float *s;
    int dt;
    int rows, cols;
    int br, bc;
    int scols;
} Glm53fMat;

/* y[rows] = M . x[cols]: per (row, column block) eight fp32 lanes of fused products, reduced
 * in double, scaled by the block scale and summed in double over blocks in order. The GPU
 * kernel reproduces this arithmetic bit for bit. */
void glm53f_mm(float *y, const float *x, const Glm53fMat *m);
/* The same product for T stacked inputs (y [T][rows], x [T][cols]); identical per token. */
void glm53f_mm_batch(float *y, const float *x, int T, const Glm53fMat *m);

static inline float glm53f_bf16f(uint16_t h)
{
    union { uint32_t u; float f; } v;
    v.u = (uint32_t)h << 16;
    return v.f;
}

/* FP8 -> GLM53F_WI4 (include/glm53f/glm53f.h:144-147, src/core/glm53f_ops.c:302-371): q holds
 * rows*(cols/2) bytes, steps rows*(cols/GLM53F_I4_GROUP) floats; per row and group of 64 columns
 * step = max|w|/7, level = rint(w/step) clamped to [-8, 7]. cols must be a multiple of 64. Runs on
 * the GPU (g53h_i4_from_f8); src, q and steps may each be host or HBM memory. */
void glm53f_i4_from_f8(unsigned char *q, float *steps, const Glm53fMat *src);

/* E4M3FN code -> float, exact; 0x7f and 0xff are NaN. */
float glm53f_e4m3f(uint8_t b);

/* y[i] = silu(min(g[i], limit)) * clamp(u[i], -limit, limit) over gu = [g | u] of 2n. */
void glm53f_swiglu_clamp(float *y, const float *gu, int n, float limit);

/* One routed expert: three FP8 (or int4) matrices. */
typedef struct {
    Glm53fMat gate, up, down;
} Glm53fExpertQ;

/* Where routed experts come from. get() returns views valid until the matching release();
 * hint() must not block and must not change what get() returns. */
typedef struct Glm53fExpertSrc {
    int (*get)(struct Glm53fExpertSrc *self, int layer, int expert, Glm53fExpertQ *out);
    int (*getmany)(struct Glm53fExpertSrc *self, int layer, const int *experts, int n);
    void (*release)(struct Glm53fExpertSrc *self, int layer, int expert);
    void (*hint)(struct Glm53fExpertSrc *self, int layer, const int *experts, int n);
    void *ctx;
} Glm53fExpertSrc;

/* One MoE layer's weights. gate is the router [n_experts][hidden] in fp32 (as the reference
 * binds it); bias is the selection bias. next_gate/next_bias predict the next layer's
 * experts for src->hint. ahead_* are carried for layout only. */
typedef struct {
    const float *gate;
    const float *bias;
    Glm53fMat    sh_gate, sh_up, sh_down;
    Glm53fExpertSrc *src;
    const float *next_gate, *next_bias;
    const float *ahead_gate[3], *ahead_bias[3];
    int          prefetch_n;
    int          prefill_next;
    int          layer;
} Glm53fMoeW;

/* Routed experts that failed to load; non-zero means the output is corrupt. */
extern long glm53f_expert_drops;
/* Non-zero silences progress lines. */
extern int glm53f_quiet;
/* Directory of int4 expert containers (include/glm53f/glm53f.h:297). Kept so that callers built
 * against the reference link; the on-disk container is outside this library, so the HBM cache in
 * int4 mode always re-quantises the FP8 experts on the device as they land. */
extern const char *glm53f_i4_dir;

/* Router: idx/w get topk entries; selection by sigmoid(W x) + bias, weights from the
 * unbiased sigmoid, renormalised if norm_topk, times routed_scale. Bit-exact with the
 * reference, including the lowest-index tie rule. */
void glm53f_router(int *idx, float *w, const float *x, const Glm53fMoeW *m, const Glm53fCfg *c);

/* Host scratch floats glm53f_moe accepts. The GPU path keeps its working set in HBM, so the
 * caller's scratch is not written; the size is reported as the reference computes it so
 * that callers that size buffers from it are unchanged. */
size_t glm53f_moe_scratch(const Glm53fCfg *c, int T);
/* out[T][hidden] = sum_j w_j expert_j(x) + shared(x). */
void   glm53f_moe(float *out, const float *x, const Glm53fMoeW *w, const Glm53fCfg *c,
                  int T, float *scratch);
/* The routed sum only (no shared expert). */
void   glm53f_moe_routed(float *out, const float *x, const Glm53fMoeW *w, const Glm53fCfg *c,
                         int T, float *scratch);

size_t glm53f_mlp_scratch(const Glm53fCfg *c);
/* Dense SwiGLU MLP: out = down(swiglu(gate x, up x)); used for the shared expert. */
void   glm53f_mlp(float *out, const float *x, const Glm53fMat *gate, const Glm53fMat *up,
                  const Glm53fMat *down, float limit, float *scratch);

/* Drop every HBM copy made of host weight pointers (router, bias, shared expert, host expert
 * views). Needed only when the caller rewrites weight bytes behind a pointer it passed. */
void   glm53f_forget_host_weights(void);

#ifdef __cplusplus
}
#endif

#endif /* GLM53F_H */
