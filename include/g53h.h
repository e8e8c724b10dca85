/* g53h.h - the thin C ABI between the C host code of the expert path and the gfx950 HIP
 * kernels. Plain pointers and sizes only; every pointer named *_d or documented as device
 * is HBM of the current device. All calls are issued on the library's compute stream and
 * are asynchronous unless stated; g53h_sync() waits. Return value 0 = success, -1 = error
 * (g53h_error() then holds the message).
 *
 * The reference has no device code for this path (its CUDA backend sends routed experts
 * back to the CPU, src/gpu/glm53f_gpu.c:1023-1041); each entry point below replaces a CPU
 * function of src/core/glm53f_ops.c, cited per declaration.
 */
#ifndef G53H_H
#define G53H_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ runtime ---- */
int         g53h_init(int device);          /* select device, create streams; idempotent */
int         g53h_device_count(void);
const char *g53h_error(void);               /* last error message ("" if none)           */
int         g53h_sync(void);                /* wait for the compute and copy streams     */
void       *g53h_alloc(size_t bytes);       /* HBM, 256-byte aligned; NULL on failure    */
int         g53h_free(void *p);
void       *g53h_host_alloc(size_t bytes);  /* pinned host memory                        */
int         g53h_host_free(void *p);
int         g53h_h2d(void *dst_d, const void *src_h, size_t bytes);   /* synchronous */
int         g53h_d2h(void *dst_h, const void *src_d, size_t bytes);   /* synchronous */
int         g53h_d2d(void *dst_d, const void *src_d, size_t bytes);   /* stream-ordered */
/* Stream-ordered copy to HBM; src must stay unchanged until the stream has passed the copy
 * (pinned host memory makes it asynchronous). */
int         g53h_h2d_async(void *dst_d, const void *src_h, size_t bytes);
/* Stream-ordered copy to the host (asynchronous into pinned memory); dst holds the bytes once
 * the stream has passed the copy (g53h_sync). */
int         g53h_d2h_async(void *dst_h, const void *src_d, size_t bytes);
int         g53h_memset(void *dst_d, int value, size_t bytes);        /* stream-ordered */
int         g53h_is_device_ptr(const void *p);   /* 1 = HBM of a device, 0 = host      */
/* Timing on the compute stream: the elapsed time between the two most recent marks. */
int         g53h_mark(void);
float       g53h_elapsed_ms(void);
/* Per-kernel timing of the layer entry points: with profiling on, each kernel launch is
 * followed by an event; g53h_prof_collect waits and returns, per tag (1 router, 2 gate/up,
 * 3 down, 4 generic path, 5 grouped path, 6 combine, 7 one-launch decode layer), the summed
 * milliseconds and the number of launches since the last collect, in arrays of ntags entries indexed by tag. */
int         g53h_prof_enable(int on);
int         g53h_prof_collect(float *ms, int *count, int ntags);
/* HBM size and free bytes of the current device. */
int         g53h_mem_info(size_t *free_b, size_t *total_b);

/* -------------------------------------------------------------- FP8 matrices ---- */
/* One FP8 E4M3 matrix in HBM: codes w, fp32 block scales s [ceil(rows/br)][scols],
 * scols = ceil(cols/bc). Field order mirrors Glm53fMat.
 *
 * Code layouts (flags bit G53H_MAT_TILED):
 *   row-major   w[r * cols + c];
 *   octet-tiled (rows a multiple of 8, cols of 128, 128-column blocks): the matrix is cut into
 *               units of 8 rows x 128 columns (1 KB), stored unit (r / 8, c / 128) at byte
 *               ((r / 8) * (cols / 128) + c / 128) * 1024, so one row octet's units follow
 *               each other. Inside a unit, row r % 8 holds 128 bytes: eight 16-byte runs, run
 *               p holding columns a, a + 8, ..., a + 120 of the block (a = g53h_tile_acc(p)).
 *               One 64-lane load of 16 bytes per lane then reads a unit whole, and each lane
 *               receives exactly the codes of one of the reference's eight per-block fp32
 *               accumulators of one row (src/core/glm53f_ops.c:185-228), in order. */
#define G53H_MAT_DROPPED 1      /* on an expert's gate: the expert failed to load             */
#define G53H_MAT_TILED   2      /* codes in the octet-tiled layout                            */
/* MFMA-tiled (rows a multiple of 8, cols of 128, 128-column blocks): the octet-tiled units,
 * with the bytes inside a unit in the operand order of the FP8 matrix cores: column
 * c = 32 g + 16 i + j (g < 4, i < 2, j < 16) of unit row m at byte i * 512 + (8 g + m) * 16 + j.
 * One 64-lane load of 16 bytes per lane reads half a unit, and lane 8 g + m of the two halves
 * holds the 32 consecutive columns 32 g .. 32 g + 31 of row m. The decode kernel k_dec_mfma
 * streams it (results within the north-star tolerance, not bit-exact). */
#define G53H_MAT_MTILED  8
/* The reference's int4 format (GLM53F_WI4, include/glm53f/glm53f.h:115-125): w holds packed
 * levels [rows][cols / 2] (element (i, j) is nibble j % 2 of byte i * cols / 2 + j / 2, the even
 * column in the low nibble, minus 8), s one fp32 step per row and group of bc columns,
 * [rows][scols]; br is ignored (one step row per matrix row). cols must be even. */
#define G53H_MAT_I4      4
/* Int4 codes (with G53H_MAT_I4) in the int4-tiled layout the one-launch int4 decode streams:
 * units of 8 rows x 256 columns (1 KB), unit (r / 8, c / 256) at ((r / 8) (cols / 256) + c / 256)
 * KB; inside a unit row m holds 128 bytes at 128 m, as 8 runs of 16: run p holds accumulator
 * g53h_tile_acc(p) of each of the block's four 64-column groups, group g in the run's bytes
 * 4 g .. 4 g + 3, level i (column 64 g + acc + 8 i) in nibble i (the low nibble first). The steps
 * stay [rows][cols / 64]. One 64-lane load of 16 bytes per lane reads a unit and leaves in each
 * lane exactly the 8 levels of one of the reference's eight fp32 accumulators of four groups. */
#define G53H_MAT_I4T     16
/* Int4 levels (G53H_MAT_I4 with G53H_MAT_MTILED) in the operand order of the FP4 matrix cores,
 * the layout of the int4 k_dec_mfma: units of 8 rows x 128 columns (512 bytes), unit (r / 8,
 * c / 128) at ((r / 8) (cols / 128) + c / 128) * 512; lane slot 8 g + m (g < 4, m < 8) of a unit
 * holds 16 bytes: row m's columns 64 (g & 1) + 16 (g >> 1) + 0..15 and then + 32 .. + 47, each
 * run as the 8 row-major bytes (the even column in the low nibble). The steps are tiled the same
 * way: 16 floats per unit at its index * 16, [64-column half of the block][row m]. One 64-lane
 * load of 16 bytes per lane reads two row octets' units of one block. */
typedef struct {
    const uint8_t *w;
    const float   *s;
    int rows, cols, br, bc, scols;
    int flags;
} G53hMat;

/* Accumulator (column offset within a 128-column block, 0..7) held by 16-byte run p of a row in
 * a tiled unit: runs 0-3 are accumulators 0, 4, 2, 6 and runs 4-7 are 1, 5, 3, 7, so that the
 * reference's pairwise tree ((a0 + a4) + (a2 + a6)) + ((a1 + a5) + (a3 + a7)) joins neighbours,
 * then pairs of neighbours, then the two halves. */
static inline int g53h_tile_acc(int p) { return ((p & 1) << 2) | (p & 2) | (p >> 2); }

/* One expert: gate [I][E], up [I][E], down [E][I]. A NULL gate.w marks an expert that
 * is not there: with G53H_MAT_DROPPED in gate.flags it could not be loaded (its contributions
 * are zero, as the reference's drop path); otherwise it is outside the current batch
 * (g53h_moe_partial). */
typedef struct {
    G53hMat gate, up, down;
} G53hExpert;

/* y[T][rows] = M . x[T][cols], bit-exact with glm53f_mm per token
 * (replaces src/core/glm53f_ops.c:185-228 matmul_f8 and :376-444 matmul_f8_batch; for a
 * G53H_MAT_I4 matrix src/core/glm53f_ops.c:236-296 matmul_i4). */
int g53h_mm_f8(float *y_d, const float *x_d, int T, const G53hMat *m);

/* FP8 -> int4 re-quantisation (replaces src/core/glm53f_ops.c:302-371 glm53f_i4_from_f8), bit-exact:
 * per row and group of 64 columns, step = max|value| / 7 (the block scale folded into the step
 * when the group lies in one scale block, else into the values; floor 1e-30), level =
 * clamp(rint(value / step), -8, 7). q_d [rows][cols / 2], steps_d [rows][cols / 64]; src is a
 * row-major FP8 matrix with cols a multiple of 64. Stream-ordered on the compute stream. NaN codes
 * (E4M3 0x7f / 0xff) give level 0 and do not count towards the maximum (the reference's scalar
 * build; its AVX2 build differs on them, and checkpoints hold none). */
int g53h_i4_from_f8(uint8_t *q_d, float *steps_d, const G53hMat *src);

/* y[T][n] = swiglu_clamp(gu[T][2n]) (replaces src/core/glm53f_ops.c:486-494). */
int g53h_swiglu(float *y_d, const float *gu_d, int n, int T, float limit);

/* Router for T tokens (replaces src/core/glm53f_ops.c:945-976 glm53f_router): idx [T][K],
 * w [T][K]. gate is [n_experts][hidden] fp32 (gate_dt 0) or bf16 bits (gate_dt 1). A token
 * whose selection finds no finite candidate sets *nan_flag_d (int, device) to 1. */
int g53h_router(int *idx_d, float *w_d, const float *x_d, int T, const void *gate_d,
                int gate_dt, const float *bias_d, int n_experts, int hidden, int topk,
                int norm_topk, float routed_scale, int *nan_flag_d);

/* Next-layer prediction (replaces src/core/glm53f_ops.c:1021-1042 route_topn): the n best
 * experts of sigmoid(W x) + bias for one token, strict order, lowest index on ties. */
int g53h_route_topn(int *idx_d, int n, const float *x_d, const void *gate_d, int gate_dt,
                    const float *bias_d, int n_experts, int hidden);

/* One decode token (T = 1): g53h_router (with *nan_flag_d written 0 or 1, no clearing needed)
 * and, when next_gate != NULL and n > 0, g53h_route_topn of the next layer's router into pred
 * [n], in two launches. Replaces src/core/glm53f_ops.c:1169-1203 (route, then route_topn for the
 * hint) for the drop-in's cached decode. With mb_slot >= 0 the kernel also writes idx [topk],
 * the flag and pred [n] as 32-bit words into the host mailbox at byte offset mb_off, then seq
 * into sequence word mb_slot (see g53h_mailbox below). */
int g53h_route_decode(int *idx_d, float *w_d, int *nan_flag_d, int *pred_d, int n, const float *x_d,
                      const void *gate_d, int gate_dt, const float *bias_d, const void *next_gate_d, int next_dt,
                      const float *next_bias_d, int n_experts, int hidden, int topk, int norm_topk,
                      float routed_scale, int mb_slot, unsigned seq, size_t mb_off);

/* route_topn for T tokens at once: idx [T][n]; score_out [T][n] (optional) receives the chosen
 * experts' sigmoid scores (for the GLM53F_ROUTE_TOP16 trace, src/core/glm53f_ops.c:1044-1080). */
int g53h_route_topn_batch(int *idx_d, float *score_out_d, int n, const float *x_d, int T, const void *gate_d,
                          int gate_dt, const float *bias_d, int n_experts, int hidden);
/* The prefill prediction's vote over ids_d [T][n] (replaces src/core/glm53f_ops.c:1206-1225):
 * out_d[0] = the number of distinct experts, out_d[1 ..] = those experts, most voted first, ties
 * in order of first appearance. out_d holds 1 + n_experts ints; n_experts <= 1024. */
int g53h_vote(int *out_d, const int *ids_d, int T, int n, int n_experts);

/* ---------------------------------------------------------------- MoE layer ---- */
typedef struct {
    int   hidden, inter, n_experts, topk, norm_topk;
    float routed_scale, swiglu_limit;
    const void       *router;       /* device [n_experts][hidden], fp32 or bf16            */
    int               router_dt;    /* 0 fp32, 1 bf16                                      */
    const float      *bias;         /* device [n_experts]                                  */
    const G53hExpert *experts;      /* device array [n_experts] of expert descriptors      */
    const G53hExpert *shared;       /* device pointer to one descriptor, or NULL           */
    int               block_c;      /* FP8 column block of every expert matrix (128 takes the
                                       tiled kernels; any other value the generic ones)     */
    int               tiled;        /* 1: every expert matrix (routed and shared) is in the
                                       octet-tiled layout (G53H_MAT_TILED), 2: MFMA-tiled
                                       (G53H_MAT_MTILED), 3: routed experts int4, int4-tiled
                                       (G53H_MAT_I4 | G53H_MAT_I4T), the shared expert FP8
                                       octet-tiled (single-token decode only; block_c 128),
                                       4: routed experts int4, int4 MFMA-tiled (G53H_MAT_I4 |
                                       G53H_MAT_MTILED), the shared expert FP8 MFMA-tiled
                                       (single-token decode by k_dec_mfma, within the
                                       tolerance; block_c 128),
                                       0: row-major                                          */
    /* Experts in the int4 format (G53H_MAT_I4, per matrix) need block_c = 0 and tiled = 0: the
       row-wave kernels then take them (and any FP8 matrix, such as the shared expert, in the
       same layer; an octet-tiled one streams fastest), exactly as glm53f_mm on a GLM53F_WI4
       matrix. */
} G53hMoeLayer;

/* Whole MoE layer on the device (replaces src/core/glm53f_ops.c:1144-1342 moe_chunk with
 * src/core/glm53f_ops.c:1344-1362 glm53f_moe / _routed): route, run the chosen experts and
 * the shared expert, combine in double in top-k order. out, x: device [T][hidden].
 * idx_d / w_d (device [T][topk]) receive the routing when non-NULL. No host round trip. */
int g53h_moe(float *out_d, const float *x_d, int T, const G53hMoeLayer *L, int *idx_d,
             float *w_d);

/* The same with the routing already done (idx_d / w_d given, device [T][topk]); used by the
 * host drop-in, which routes first to fetch the experts through an Glm53fExpertSrc. */
int g53h_moe_routed_given(float *out_d, const float *x_d, int T, const G53hMoeLayer *L,
                          const int *idx_d, const float *w_d);

/* Partial layer for a host driver that fetches experts in batches (the drop-in path):
 * contributions of the slots whose expert descriptor is present go to contrib_d
 * [T][topk + has_shared][hidden]; slots whose descriptor has gate.w == NULL are left
 * untouched, except that a descriptor marked G53H_MAT_DROPPED (a dropped expert) writes zeros.
 * g53h_moe_combine then forms out = (float)(sum_j w_j contrib_j in double) (+ shared). */
int g53h_moe_partial(float *contrib_d, const float *x_d, int T, const G53hMoeLayer *L,
                     const int *idx_d);
int g53h_moe_combine(float *out_d, const float *contrib_d, const float *w_d, int T,
                     const G53hMoeLayer *L);

/* Batched decode and prefill (T >= 2) as token-sorted grouped GEMMs on the FP8 matrix cores
 * (row-major experts, or octet-tiled ones when L->tiled: every expert matrix, routed and shared,
 * in the layout L->tiled names; a descriptor of the other layout counts as unusable, flag 8)
 * (replaces src/core/glm53f_ops.c:1144-1342 moe_chunk with :376-444 matmul_f8_batch for a chunk
 * of tokens): every expert's weights are read once per call of up to 2048 tokens. Routing is the
 * exact router's (top-k indices and weights bit-exact); the expert products run on
 * v_mfma_scale_f32_32x32x64_f8f6f4 with the activations split into E4M3 planes, so outputs
 * match the reference within 2e-3 relative + 1e-2 absolute rather than bit for bit. Layers need
 * 128x128 blocks, hidden and inter multiples of 512 with power-of-two block counts up to 32,
 * topk <= 16, at most 1024 experts and a finite positive SwiGLU limit (g53h_grouped_ok).
 * g53h_moe takes this path for T >= 2 when g53h_set_grouped is on (the default; it returns the
 * previous setting) and the layer qualifies; otherwise the exact per-token kernels.
 * g53h_grouped_errors waits for the stream and returns, then clears, the grouped kernels' flags
 * (1: a routed index out of range, 2: a wait between waves timed out, 8: an expert descriptor
 * without the 128x128 layout). */
int g53h_moe_grouped(float *out_d, const float *x_d, int T, const G53hMoeLayer *L, int *idx_d,
                     float *w_d);
/* The grouped layer in phases, for a host driver that fetches experts in batches (the C
 * drop-in; replaces the expert loop of src/core/glm53f_ops.c:1240-1340 for a chunk of tokens):
 * begin plans T <= g53h_grouped_max_tokens(L) tokens with the routing given (idx_d
 * [T][topk]) and splits x; each batch call multiplies the experts whose descriptors in
 * L->experts (and L->shared) are present, leaves the others for other batches, and gives zero
 * contributions to descriptors marked dropped (gate.w == NULL, G53H_MAT_DROPPED); end combines
 * into out_d with the weights w_d [T][topk]. Between begin and end the library's workspace
 * holds the pass: no other g53h layer call may run in between (copies may). */
int g53h_grouped_max_tokens(const G53hMoeLayer *L);   /* 0: the layer's shapes do not qualify */
int g53h_grouped_begin(const float *x_d, int T, const G53hMoeLayer *L, const int *idx_d);
int g53h_grouped_batch(const G53hMoeLayer *L);
int g53h_grouped_end(float *out_d, const float *w_d);
int g53h_set_grouped(int on);
int g53h_grouped_ok(const G53hMoeLayer *L);
int g53h_grouped_errors(void);
/* Diagnostics: with dev_buf != NULL (device, at least (gate/up items) x 8 uint64), the grouped
 * gate/up kernel records 100 MHz timestamps of each item's phases; NULL turns it off. */
int g53h_set_grouped_trace(void *dev_buf);

/* Single-token decode runs as one persistent launch when the layer has the released shapes
 * (hidden 4096, inter 2048, 128x128 blocks, topk <= 15): k_dec_tiled for a layer whose experts
 * are octet-tiled (L->tiled), k_dec_layer for row-major ones; g53h_set_fused_decode(0) selects
 * the multi-kernel path instead (returns the previous setting). g53h_decode_errors waits for the
 * stream and returns, then clears, the fused kernel's error flags (1: a grid wait timed out,
 * 2: a token had fewer than topk selectable experts, 8: an unusable expert descriptor, which
 * then contributes zero), 0 if none. g53h_decode_grid returns the
 * fused kernel's workgroup count (0: unavailable, -1: not yet sized). */
int g53h_set_fused_decode(int on);

/* No counterpart in the reference: single-token decode that allocates nothing, for callers
 * that cannot call hipMalloc (code under HIP graph capture, serving loops, harnesses that
 * forbid it). Same result as g53h_moe at T = 1 through k_dec_tiled, bit for bit; the layer must
 * be one that kernel takes (octet-tiled experts, hidden 4096, inter 2048, 128-column blocks,
 * bf16 router), with n_experts <= 1024 and topk <= 15, else it fails with an error. Its scratch
 * (tagged scores and activations, 4.2 MB) is a fixed device array each device holds until the
 * process ends, set up by g53h_init; calls that overlap on one device race. out, x: device
 * [hidden]; idx_d / w_d (device [topk]) receive the routing when non-NULL. */
int g53h_moe_decode_noalloc(float *out_d, const float *x_d, const G53hMoeLayer *L, int *idx_d, float *w_d);
int g53h_decode_errors(void);
int g53h_decode_grid(void);
/* Error flags of the layer kernels, for a caller that reads them with its own synchronisation
 * (the C drop-in): enqueues on the compute stream a copy of the G53H_NERR flag words into
 * host (pinned memory keeps the copy asynchronous), then clears them; host holds them once the
 * stream has passed that point. [0] k_dec_layer and [1] k_dec_tiled (the bits of
 * g53h_decode_errors), [2] the grouped path (the bits of g53h_grouped_errors). */
#define G53H_NERR 3
int g53h_errors_async(int *host);
/* The same copy without clearing the flags: for a caller that aborts on any flag (the C drop-in),
 * so that nothing needs clearing while no flag is set. */
int g53h_errors_peek_async(int *host);
/* Host mailbox: G53H_MBOX_BYTES of pinned host memory that kernels write into directly, so a
 * host waits for a result by polling a word instead of a device-to-host copy and a stream
 * synchronisation. Words [0, G53H_MBOX_SLOTS) are sequence words; data lives above them.
 * g53h_mailbox_wait spins until sequence word `slot` equals seq (then the data written before
 * it is visible), falling back to a blocking stream wait. g53h_publish enqueues on the compute
 * stream a copy of the G53H_NERR error words and then `bytes` of device memory into the mailbox
 * at byte offset off, followed by seq in word `slot`. */
#define G53H_MBOX_BYTES (1 << 16)
#define G53H_MBOX_SLOTS 16
void *g53h_mailbox(void);
int   g53h_mailbox_wait(int slot, unsigned seq);
/* The inbox, the other direction: G53H_INBOX_BYTES of pinned, mapped host memory that kernels
 * read. g53h_inbox_fetch enqueues on the compute stream a kernel that copies bytes (a multiple
 * of 16, at a multiple of 16) of it into device memory, so that small inputs reach the stream
 * without the copy engine. The host must not rewrite those bytes before the stream has passed
 * the fetch (a later wait on it). */
#define G53H_INBOX_BYTES (1 << 16)
void *g53h_inbox(void);
int   g53h_inbox_fetch(void *dst_d, size_t off, size_t bytes);
int   g53h_publish(int slot, unsigned seq, size_t off, const void *src_d, size_t bytes);

/* The next layer's router scores for one decode token (the scores of
 * src/core/glm53f_ops.c:1190-1228's prediction: sigmoid of next_gate . x, plus next_bias for the
 * choice), kept in a library buffer for g53h_decode_publish. n_experts <= 1024. */
int   g53h_route_next(const float *x_d, const void *next_gate_d, int next_dt, const float *next_bias_d,
                      int n_experts, int hidden);
/* The same scores requested of the next single-token decode launch: the octet-tiled one-launch
 * decode computes them with its spare waves when the router is bf16 and they fit (n_experts <=
 * 2 x its grid), else g53h_decode_publish launches g53h_route_next itself. x_d must stay
 * unchanged until then. */
int   g53h_decode_next(const float *x_d, const void *next_gate_d, int next_dt, const float *next_bias_d,
                       int n_experts, int hidden);
/* One launch after a decode layer: the next layer's top-n from the last g53h_route_next (n = 0:
 * none; into pred_d [n]), then into the mailbox idx_d [topk], the NaN flag (bit 2 of the decode
 * error words) and pred [n] as 32-bit words at route_off, the G53H_NERR error words and
 * out_bytes of out_d at out_off, and seq into sequence word `slot` (g53h_route_decode and
 * g53h_publish in one, after a layer kernel that routed by itself). */
int   g53h_decode_publish(int slot, unsigned seq, size_t route_off, const int *idx_d, int topk, int *pred_d,
                          int n, int n_experts, size_t out_off, const void *out_d, size_t out_bytes);

/* Test hook: the number of polls after which a wait on another workgroup of the one-launch
 * decode kernels gives up (and sets bit 1 of their error flags); 0 restores the default.
 * Returns the previous setting. Waits between the waves of one workgroup are not affected. */
int g53h_set_spin_limit(int polls);
/* Test hook: ORs bits into error word `word` (0 .. G53H_NERR-1) on the compute stream, as a
 * kernel that hit that condition would; the caller's next read of the flags sees them. */
int g53h_inject_errors(int word, int bits);
/* Diagnostics: with dev_buf != NULL (device, grid x 32 uint64), the fused kernel's workgroups
 * record 100 MHz timestamps at their phase boundaries; NULL turns it off. */
int g53h_set_decode_trace(void *dev_buf);
int g53h_set_tiled_decode_trace(void *dev_buf);   /* the same for the octet-tiled kernel   */
int g53h_set_mfma_decode_trace(void *dev_buf);    /* the same for the MFMA-tiled kernel    */

/* ------------------------------------------------------------- code layouts ---- */
/* Row-major FP8 codes [rows][cols] -> octet-tiled (see G53hMat), and back; stream-ordered on
 * the compute stream, dst and src distinct, rows a multiple of 8 and cols of 128. The host
 * twin converts in host memory (inverse != 0: tiled -> row-major). */
int g53h_tile_f8(uint8_t *dst_d, const uint8_t *src_d, int rows, int cols);
int g53h_untile_f8(uint8_t *dst_d, const uint8_t *src_d, int rows, int cols);
int g53h_tile_f8_host(uint8_t *dst, const uint8_t *src, int rows, int cols, int inverse);
/* The same for the MFMA-tiled layout (G53H_MAT_MTILED); inverse != 0 converts back. */
int g53h_mtile_f8(uint8_t *dst_d, const uint8_t *src_d, int rows, int cols, int inverse);
int g53h_mtile_f8_host(uint8_t *dst, const uint8_t *src, int rows, int cols, int inverse);
/* Int4 levels [rows][cols / 2] (row-major, the reference's GLM53F_WI4) to the int4-tiled layout
 * (G53H_MAT_I4T); inverse != 0 converts back. rows a multiple of 8, cols of 256. */
int g53h_tile_i4(uint8_t *dst_d, const uint8_t *src_d, int rows, int cols, int inverse);
int g53h_tile_i4_host(uint8_t *dst, const uint8_t *src, int rows, int cols, int inverse);
/* Int4 levels [rows][cols / 2] and steps [rows][cols / 64] (GLM53F_WI4) to the int4 MFMA-tiled
 * layout (G53H_MAT_I4 | G53H_MAT_MTILED), levels and steps together; inverse != 0 converts back.
 * rows a multiple of 8, cols of 128; the host twin skips the steps when either is NULL. */
int g53h_mtile_i4(uint8_t *dst_w, float *dst_s, const uint8_t *src_w, const float *src_s, int rows, int cols,
                  int inverse);
int g53h_mtile_i4_host(uint8_t *dst_w, float *dst_s, const uint8_t *src_w, const float *src_s, int rows, int cols,
                       int inverse);

/* -------------------------------------------------------- checks and inputs ---- */
/* y[i] = expf(x[i]) by the device restatement of glibc's expf (for exhaustive checks). */
int g53h_expf(float *y_d, const float *x_d, size_t n);
/* y[i] = expf of the float whose bit pattern is base + i, i < n (no input buffer). */
int g53h_expf_range(float *y_d, uint32_t base, size_t n);
/* Host twin of the device expf restatement (the same source compiled for the CPU). */
void g53h_expf_host(float *y, const float *x, size_t n);
/* out[i] = E4M3 code[i] decoded by the gfx950 conversion instruction the kernels use. */
int g53h_e4m3_decode(float *out_d, const uint8_t *codes_d, size_t n);

/* Seeded synthetic FP8 matrix: element (i,j) ~ N(0, sigma^2) from (seed, stream, i*cols+j),
 * quantised per br x bc block by the absmax rule. The host twin g53h_synth_f8_host gives the
 * same bytes on the CPU. */
int  g53h_synth_f8(uint8_t *w_d, float *s_d, int rows, int cols, int br, int bc,
                   uint64_t seed, uint64_t stream, float sigma);
void g53h_synth_f8_host(uint8_t *w, float *s, int rows, int cols, int br, int bc,
                        uint64_t seed, uint64_t stream, float sigma);
/* n values N(0, sigma^2) (host); as bf16 bit patterns widened to float when bf16 != 0. */
void g53h_synth_normal_host(float *out, size_t n, uint64_t seed, uint64_t stream, float sigma,
                            int bf16);
/* q[i] = E4M3(clamp(x[i] * scale, +-448)), the generator's quantiser (host). */
void g53h_quant_host(uint8_t *q, const float *x, size_t n, float scale);
/* n values U(-a, a) (host). */
void g53h_synth_uniform_host(float *out, size_t n, uint64_t seed, uint64_t stream, float a);

#ifdef __cplusplus
}
#endif

#endif /* G53H_H */
