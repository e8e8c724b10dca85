/* glm53f_cache.h - the routed-expert cache, in HBM, with predictive prefetch from host memory.
 *
 * Drop-in for the reference's src/cache/glm53f_cache.h:99-103 (glm53f_cache_init/free/
 * reset_stats/report) and its Glm53fCache whose first member is the Glm53fExpertSrc the MoE
 * layer reads experts through (src/cache/glm53f_cache.h:45). Same policy as the reference
 * (src/cache/glm53f_cache.c): LRU over fixed slots, a slot is never handed out while pinned
 * (between get() and release()) or while a read into it is being set up; hint() queues the
 * experts a layer will need, ordered by layer, and cancels stale entries; prefetch changes
 * only what is resident when, never what get() returns.
 *
 * What is different on MI355X:
 *   - the slots are HBM (a slot holds one expert's FP8 codes and block scales) and get()
 *     returns DEVICE views: pass them to the library's kernels (glm53f_moe does);
 *   - a missing expert is copied from the store's host memory (pinned for full PCIe speed) with
 *     hipMemcpyAsync on a copy stream; the library's compute stream waits for that copy with
 *     a stream event, so get() does not block the host;
 *   - release() records an event on the compute stream; a later copy into the same slot waits
 *     for it on the copy stream, so a slot is never overwritten while a kernel still reads it;
 *   - n_io is the number of prefetch copies kept in flight (0 disables prefetch), instead of a
 *     number of I/O threads;
 *   - glm53f_cache_init reads experts from the checkpoint index (Glm53fSt, the reference's
 *     reader type): each missing expert is read from its shard into a pinned staging buffer
 *     (two reads when its three weights and its three scale grids each lie in one run, as
 *     the released checkpoint stores them, else six), then copied to the slot;
 *   - g53h_cache_init_store takes any other source of host-resident experts (G53hStore
 *     below), e.g. experts already in pinned host memory;
 *   - int4 slots (i4 != 0, the reference's --experts int4): each FP8 expert read is staged in
 *     HBM and re-quantised into the slot by the device quantiser (g53h_i4_from_f8, bit-exact
 *     with the reference's glm53f_i4_from_f8), in the reference's int4 slot layout, so a budget
 *     holds the reference's number of slots and get() returns its GLM53F_WI4 views. The
 *     reference's on-disk int4 container (glm53f_i4_dir) is not read: every layer is quantised
 *     on the way in, and i4_layers stays zero.
 */
#ifndef GLM53F_CACHE_H
#define GLM53F_CACHE_H

#include <pthread.h>
#include <stdint.h>

#include "glm53f.h"
#include "glm53f_st.h"
#include "g53h.h"

#ifdef __cplusplus
extern "C" {
#endif

#define GLM53F_SLOT_EMPTY     (-1)
#define GLM53F_SLOT_INFLIGHT  (-2)

/* The reference's cache struct (src/cache/glm53f_cache.h:44-96), field for field, so that its
 * callers (the model code reads nslot, slot_bytes, i4_layers and the statistics, and passes
 * &cache.src to the MoE layers) compile and read the right values unchanged. What each field
 * holds here:
 *   src                the expert source (get/getmany/release/hint) over the HBM slots
 *   st, cfg            as given to glm53f_cache_init (st is NULL for g53h_cache_init_store)
 *   arena              the HBM slot arena (a device pointer), nslot slots of slot_bytes
 *   slot_of ... used_at, clock, qcap, qlen, hint_floor, last_hint, queued
 *                      the LRU bookkeeping, with the reference's meaning (read-only for
 *                      callers; clock is refreshed at each call)
 *   n_io               prefetch copies kept in flight (0: prefetch off)
 *   stage              this library's state (an opaque pointer; the int4 staging it names in
 *                      the reference lives in HBM here, inside that state)
 *   i4                 1 for int4 slots
 *   statistics         as the reference's, reset by glm53f_cache_reset_stats
 * Unused here, left zero: raw_bytes, stage_busy, nstage, stage_free, i4_fd, i4_layers, ref,
 * pad, mu, landed, work, io, stop, queue. */
typedef struct {
    Glm53fExpertSrc  src;             /* MUST be first: pass &cache->src to Glm53fMoeW */

    const Glm53fSt  *st;
    const Glm53fCfg *cfg;
    int              n_layers, n_experts;

    unsigned char   *arena;
    int64_t          slot_bytes;
    int              nslot;

    int              i4;
    int64_t          raw_bytes;
    unsigned char  **stage;
    unsigned char   *stage_busy;
    int              nstage;
    pthread_cond_t   stage_free;
    int             *i4_fd;
    int              i4_layers;

    int32_t         *slot_of;         /* [n_layers*n_experts] -> resident slot, or -1  */
    int32_t         *inflight_of;     /* [n_layers*n_experts] -> slot being read, or -1 */
    int32_t         *key_of;          /* [nslot] -> key, EMPTY or INFLIGHT             */
    int32_t         *pins;            /* [nslot] experts in use                        */
    unsigned char   *prefetched;      /* [nslot] loaded by prefetch and not yet used    */
    uint64_t        *used_at;         /* [nslot] LRU stamp                             */
    void            *ref;             /* Glm53fExpertRef * in the reference; unused     */
    int64_t         *pad;
    uint64_t         clock;

    pthread_mutex_t  mu;
    pthread_cond_t   landed;
    pthread_cond_t   work;

    int              n_io;
    pthread_t       *io;
    int              stop;
    int32_t         *queue;
    int              qcap, qlen;
    int              hint_floor, last_hint;
    unsigned char   *queued;          /* [n_layers*n_experts] */

    uint64_t         hits, misses, evictions, bytes_read, prefetch_reads;
    double           load_seconds;    /* host time spent in get()/getmany()              */
    uint64_t         bg_reads, bg_bytes, bg_used;
} Glm53fCache;

/* budget_bytes is the HBM arena, rounded down to whole experts. Experts are read from the
 * checkpoint index st (tensor names "model.language_model.layers.L.mlp.experts.E.{gate,up,
 * down}_proj.{weight,weight_scale_inv}", FP8 E4M3 codes with F32 scale grids); the slot geometry
 * comes from expert 0 of the first MoE layer (cfg->is_dense), as the reference probes it.
 * Fails (-1) if fewer than topk+1 slots fit, if HBM cannot hold the arena, if the probe expert
 * is missing or not FP8, or (i4 != 0) if a matrix's columns are not a multiple of 64.
 * i4 = 1 is the reference's int4 mode (its slot layout, GLM53F_WI4 views). i4 = 2, this
 * library's own, holds the same slot size with the levels int4-tiled (GLM53F_WI4T views) at the
 * shapes the one-launch decode reads (hidden 4096, inter 2048, 128 x 128 FP8 blocks), so that
 * the drop-in decodes a token in one launch; its chunked paths untile the views they read. At
 * other shapes i4 = 2 is i4 = 1. i4 = 3, also this library's own, is i4 = 2 with levels and
 * steps int4 MFMA-tiled (GLM53F_WI4M views): the drop-in then decodes a token in one launch on
 * the FP4 matrix cores, within the path's tolerance instead of bit for bit. With the environment
 * variable GLM53F_CACHE_MFMA set to a non-zero number at init, FP8 slots at those shapes are
 * MFMA-tiled (GLM53F_WF8M views) and the drop-in decodes on the FP8 matrix cores, within the
 * tolerance. */
int  glm53f_cache_init(Glm53fCache *c, const Glm53fSt *st, const Glm53fCfg *cfg, int64_t budget_bytes,
                       int n_io, int i4);
void glm53f_cache_free(Glm53fCache *c);
void glm53f_cache_reset_stats(Glm53fCache *c);
void glm53f_cache_report(const Glm53fCache *c, const char *label);

/* Another source of host-resident experts. view() fills host views of the expert's three FP8
 * matrices (codes and fp32 scales, GLM53F_WF8) and returns 0, or -1 when the expert cannot be
 * read (get() then fails: a dropped expert). The bytes must stay valid until done() is called
 * for that expert (when the copy to HBM has completed); done may be NULL for a store whose
 * bytes never move. Calls come from the thread that calls the cache. */
typedef struct G53hStore {
    int  (*view)(const struct G53hStore *st, int layer, int expert, Glm53fExpertQ *host);
    void (*done)(const struct G53hStore *st, int layer, int expert);
    void *ctx;
} G53hStore;

/* glm53f_cache_init over a G53hStore instead of a checkpoint (no counterpart in the
 * reference, whose cache always reads the checkpoint). */
int  g53h_cache_init_store(Glm53fCache *c, const G53hStore *store, const Glm53fCfg *cfg, int64_t budget_bytes,
                           int n_io, int i4);

/* Wait until every copy the cache issued has landed (tests and benchmarks). */
int  glm53f_cache_sync(Glm53fCache *c);
/* 1 when src is the expert source of a cache made by glm53f_cache_init (its views are HBM and
 * its release is ordered on the device), else 0. */
int  g53h_cache_is(const Glm53fExpertSrc *src);
/* The device table of layer's experts whose reads have landed (no counterpart in the
 * reference): table_d [n_experts] of the slots' descriptors (octet-tiled FP8 or int4-tiled;
 * gate.w NULL where the expert holds no landed slot) on the compute stream's timeline, and table_h its host copy. It is current as
 * of this call; any later cache call may evict or fill slots, so a kernel that reads it must
 * complete before the next cache call. Returns 0, a positive count of this layer's reads still
 * in flight (no table then), or -1 when src is not a cache with tiled slots (kind 1 to 4). */
int  g53h_cache_layer_table(Glm53fExpertSrc *src, int layer, const G53hExpert **table_d,
                            const G53hExpert **table_h);
/* The kind of slots a cache holds (no counterpart in the reference): 1 octet-tiled FP8, 2
 * MFMA-tiled FP8 (GLM53F_CACHE_MFMA set at its init), 3 int4-tiled (int4 mode 2), 4 int4
 * MFMA-tiled (int4 mode 3), 0 otherwise (row-major FP8 or int4, or src not a cache). */
int  g53h_cache_slot_kind(const Glm53fExpertSrc *src);
/* The drop-in's speculative cached decode (no counterpart in the reference): with a cache of
 * octet-tiled slots, glm53f_moe at T = 1 runs the one-launch decode over the layer's table
 * before the reference's hint/get/release calls, which it then makes in the reference's order,
 * and runs the layer again only when a chosen expert had no landed slot. on = 0 makes every
 * layer route first and fetch before it computes. The environment variable G53H_NO_SPECULATE
 * sets the default to 0. It also clears the record of recent outcomes by which a layer decides
 * whether to speculate. Returns the previous setting. */
int  g53h_set_speculate(int on);
/* Counts of cached single-token layers since the last call: out[0] finished by the speculative
 * launch, out[1] speculative and run again, out[2] not speculative. Resets them. */
void g53h_speculate_counts(int64_t *out);

/* A store of experts in pinned host memory built by the library: n_pool distinct experts
 * generated from the seeded synthetic distribution (FP8 E4M3, N(0, sigma^2) absmax-quantised
 * per 128 x 128 block) of the given shapes; expert (layer, e) is pool entry
 * (layer * n_experts + e) % n_pool. For benchmarks and tests that need more experts than host
 * memory holds distinct copies of. */
int  g53h_store_synth_init(G53hStore *st, int hidden, int inter, int n_layers, int n_experts, int n_pool,
                           uint64_t seed, float sigma);
void g53h_store_synth_free(G53hStore *st);
/* Gives every (layer, expert) key of a synthetic store its own block scales: the pool entry's
 * scales times 1 + (key + 1) 2^-14, held in pinned memory (6 KB per key at the released
 * shapes), so no two keys share a payload and a slot handed back for the wrong key changes the
 * result. Call once, after g53h_store_synth_init. */
int  g53h_store_synth_key_scales(G53hStore *st);

/* The LRU policy alone on a scripted trace (CPU, no device): ops are
 *   1 L E        get          -> out: rc, was resident (1/0), slot
 *   2 L E        release
 *   3 L n e...   getmany      -> out: rc
 *   4 L n e...   hint         -> out: queue length, then the queued keys
 *   5 k          serve up to k queued hints as background reads -> out: (key, slot) per read, -1
 * and stats receives hits, misses, evictions, prefetch_reads, bg_reads, bg_used. Returns the
 * number of ints written to out, or -1. For checking the policy against the reference. */
int  g53h_lru_trace(int n_layers, int n_experts, int nslot, const int *ops, int nops, int *out, int outcap,
                    long long *stats);

#ifdef __cplusplus
}
#endif

#endif /* GLM53F_CACHE_H */
