/* g53h_cache.hip - the routed-expert cache in HBM (include/glm53f_cache.h).
 *
 * Policy: g53h_lru.c, the reference's (src/cache/glm53f_cache.c). Data movement, MI355X style:
 *   - a slot is one expert's FP8 codes and fp32 block scales in one HBM arena;
 *   - a read is six hipMemcpyAsync from the store's host memory into the slot, on the demand
 *     copy stream (get/getmany) or the prefetch copy stream (hint), followed by the slot's
 *     `landed` event. The bookkeeping publishes the slot when the copies are issued: get()
 *     makes the library's compute stream wait for `landed`, so no host thread blocks on a
 *     read (the reference waits on a condition variable instead);
 *   - release() records a `used` event on the compute stream (one event for all releases
 *     between two get() calls: the caller launched the kernels that read those slots before
 *     releasing them); a later read into the slot first waits for it (and for the slot's
 *     previous `landed`, which may be on the other copy stream), so a slot is never
 *     overwritten while a kernel still reads it. A `landed` event seen complete is not
 *     waited on again;
 *   - prefetch keeps at most n_io expert reads in flight on the prefetch stream; the queue
 *     (ordered by layer, stale entries cancelled by later hints) feeds it whenever the cache is
 *     called and earlier reads have landed.
 *   - int4 slots (i4 != 0, the reference's --experts int4): a read copies each FP8 matrix and
 *     its scales into the stream's staging buffer in HBM, and the quantiser kernel writes the
 *     slot's GLM53F_WI4 levels and steps from there on the same stream (the reference
 *     quantises on its I/O threads, src/cache/glm53f_cache.c:114-127); the slot layout is the
 *     reference's (src/io/glm53f_load.c:141-163), so a budget holds the same number of slots.
 *     In int4 mode 2 the levels are quantised into staging and int4-tiled into the slot (the
 *     same bytes per slot), for the one-launch int4 decode.
 * Every entry point takes one mutex, as the reference's. */
#include <hip/hip_runtime.h>

#include <mutex>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <vector>

#include "g53h.h"
#include "g53h_runtime.h"
#include "glm53f.h"
#include "glm53f_cache.h"
#include <unistd.h>
extern "C" {
#include "../host/g53h_ckpt.h"
#include "../host/g53h_lru.h"
}

namespace {

struct Geom {                       /* slot layout, from the probe expert */
    size_t off[6], bytes[6];        /* gate/up/down codes, then gate/up/down scales (in the slot) */
    size_t fbytes[6];               /* the same parts as read (FP8), for int4 slots            */
    int rows[3], cols[3], br[3], bc[3], scols[3];
};

struct Copy {
    hipEvent_t ev;
    int layer, expert, background, slot;
    uint64_t gen;                   /* the slot's read generation this copy filled            */
};

struct Impl {
    G53hLru lru;
    const G53hStore *store = nullptr;       /* host experts from a caller's store, or       */
    G53hCkpt *ckpt = nullptr;               /* ... read from the checkpoint into staging    */
    uint8_t *arena = nullptr;
    Geom geo;
    std::vector<hipEvent_t> landed;
    std::vector<unsigned char> landed_ok;   /* landed[slot] may still be pending            */
    std::vector<uint64_t> gen;              /* reads issued into each slot                  */
    std::vector<int> used;                  /* the slot's last release: index into used_ev, -1 */
    std::vector<hipEvent_t> used_ev;        /* release events, shared by a batch's releases */
    std::vector<int> used_refs;
    std::vector<int> used_free;
    int cur_used = -1;                      /* event recorded since the last get(), or -1   */
    hipStream_t demand = nullptr, prefetch = nullptr;
    /* octet-tiled slots (G53H_MAT_TILED): a matrix's codes land in the stream's staging buffer and
     * are tiled into the slot by a kernel on the same stream, so one buffer per stream suffices */
    bool tiled = false;
    bool mt = false;                /* with tiled: FP8 slots MFMA-tiled (GLM53F_CACHE_MFMA)  */
    bool i4 = false;                /* int4 slots: FP8 staged, quantised into the slot      */
    bool i4t = false;               /* int4 mode 2: the levels quantised into staging, then
                                       int4-tiled into the slot (the steps straight in)     */
    bool i4m = false;               /* int4 mode 3: levels and steps quantised into staging,
                                       then int4 MFMA-tiled into the slot together          */
    uint8_t *stage_demand = nullptr, *stage_prefetch = nullptr;
    size_t stage_lv = 0;            /* int4 modes 2, 3: the levels' offset in a staging buffer */
    size_t stage_st = 0;            /* int4 mode 3: the steps' offset                       */
    std::vector<Copy> inflight;     /* copies not yet seen complete                         */
    std::vector<hipEvent_t> pool;   /* spare events                                         */
    /* tiled slots: the descriptor of every key whose read has been seen complete, per layer in
     * pinned host memory (zero where the key holds no landed slot) and its device copy, which is
     * uploaded on the compute stream when the layer's entries have changed; a one-launch decode
     * that routes by itself reads its chosen experts from it */
    G53hExpert *tab_h = nullptr, *tab_d = nullptr;
    std::vector<unsigned char> tab_dirty;   /* per layer: tab_h differs from tab_d       */
    std::vector<int> tab_key;               /* per slot: the key whose entry names it, -1  */
    std::vector<int> pend;                  /* per layer: reads issued, not yet seen complete */
    std::mutex mu;
    ~Impl()
    {
        g53h_ckpt_free(ckpt);
    }
};

double now_s()
{
    timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t.tv_sec + t.tv_nsec * 1e-9;
}

size_t al(size_t v, size_t a) { return (v + a - 1) / a * a; }

size_t scale_bytes(const Glm53fMat &m) { return (size_t)((m.rows + m.br - 1) / m.br) * m.scols * sizeof(float); }

/* The library's state rides in the reference struct's int4-staging pointer, unused here. */
Impl *impl_of(const Glm53fCache *c) { return (Impl *)(void *)c->stage; }

int store_view(Impl *m, int layer, int expert, Glm53fExpertQ *h)
{
    if (m->ckpt) return g53h_ckpt_view(m->ckpt, layer, expert, h);
    return m->store->view(m->store, layer, expert, h);
}

void store_done(Impl *m, int layer, int expert)
{
    if (m->ckpt) g53h_ckpt_done(m->ckpt, layer, expert);
    else if (m->store->done) m->store->done(m->store, layer, expert);
}

void sync_stats(Glm53fCache *c, const Impl *m)
{
    c->hits = m->lru.hits;
    c->misses = m->lru.misses;
    c->evictions = m->lru.evictions;
    c->prefetch_reads = m->lru.prefetch_reads;
    c->bg_reads = m->lru.bg_reads;
    c->bg_used = m->lru.bg_used;
    c->clock = m->lru.clock;
    c->qlen = m->lru.qlen;
    c->hint_floor = m->lru.hint_floor;
    c->last_hint = m->lru.last_hint;
}

/* Drop a slot's reference to its release event. */
void unuse(Impl *m, int slot)
{
    const int u = m->used[slot];
    if (u < 0) return;
    m->used[slot] = -1;
    if (--m->used_refs[u] == 0 && u != m->cur_used) m->used_free.push_back(u);
}

void view_of(const Glm53fCache *c, const Impl *m, int slot, Glm53fExpertQ *q);

/* The descriptor table: slot's entry (its key's) cleared before the slot is read into again, and
 * set once its read has been seen complete. */
void table_clear(Glm53fCache *c, Impl *m, int slot)
{
    if (!m->tab_h || m->tab_key[slot] < 0) return;
    const int key = m->tab_key[slot];
    memset(&m->tab_h[key], 0, sizeof(G53hExpert));
    m->tab_dirty[key / c->n_experts] = 1;
    m->tab_key[slot] = -1;
}

void table_set(Glm53fCache *c, Impl *m, int slot, int layer, int expert)
{
    if (!m->tab_h) return;
    table_clear(c, m, slot);
    Glm53fExpertQ q;
    view_of(c, m, slot, &q);
    const int key = layer * c->n_experts + expert;
    G53hExpert &e = m->tab_h[key];
    G53hMat *d[3] = {&e.gate, &e.up, &e.down};
    const Glm53fMat *v[3] = {&q.gate, &q.up, &q.down};
    for (int i = 0; i < 3; i++) {
        d[i]->w = (const uint8_t *)v[i]->w; d[i]->s = v[i]->s;
        d[i]->rows = v[i]->rows; d[i]->cols = v[i]->cols; d[i]->br = v[i]->br; d[i]->bc = v[i]->bc;
        d[i]->scols = v[i]->scols;
        d[i]->flags = m->i4t ? (G53H_MAT_I4 | G53H_MAT_I4T) : m->i4m ? (G53H_MAT_I4 | G53H_MAT_MTILED)
                      : m->mt ? G53H_MAT_MTILED : G53H_MAT_TILED;
    }
    m->tab_key[slot] = key;
    m->tab_dirty[layer] = 1;
}

/* Copies seen complete hand their host bytes back to the store, and the slot they filled no
 * longer needs its landed event waited on. */
void poll(Glm53fCache *c, Impl *m)
{
    size_t k = 0;
    for (size_t i = 0; i < m->inflight.size(); i++) {
        Copy &cp = m->inflight[i];
        if (hipEventQuery(cp.ev) == hipSuccess) {
            store_done(m, cp.layer, cp.expert);
            if (m->gen[cp.slot] == cp.gen) {
                m->landed_ok[cp.slot] = 0;
                table_set(c, m, cp.slot, cp.layer, cp.expert);
            }
            if (m->tab_h) m->pend[cp.layer]--;
            m->pool.push_back(cp.ev);
        } else {
            m->inflight[k++] = cp;
        }
    }
    m->inflight.resize(k);
}

bool same_mat(const Glm53fMat &h, const Geom &g, int i)
{
    return h.dt == GLM53F_WF8 && h.w && h.s && h.rows == g.rows[i] && h.cols == g.cols[i] && h.br == g.br[i] &&
           h.bc == g.bc[i] && h.scols == g.scols[i];
}

int issue_reads(Glm53fCache *c, Impl *m, int slot, int layer, int expert, hipStream_t s, int64_t *nread);

/* Read expert (layer, expert) into slot on stream s. Returns 1 on success. */
int issue(Glm53fCache *c, Impl *m, int slot, int layer, int expert, hipStream_t s, int background, int64_t *nread)
{
    *nread = 0;
    if (!issue_reads(c, m, slot, layer, expert, s, nread)) {
        return 0;
    }
    if (hipEventRecord(m->landed[slot], s) != hipSuccess) return 0;
    m->landed_ok[slot] = 1;
    m->gen[slot]++;
    hipEvent_t ev;
    if (!m->pool.empty()) { ev = m->pool.back(); m->pool.pop_back(); }
    else if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) return 0;
    if (hipEventRecord(ev, s) != hipSuccess) return 0;
    m->inflight.push_back(Copy{ev, layer, expert, background, slot, m->gen[slot]});
    if (m->tab_h) m->pend[layer]++;
    return 1;
}

/* The reads of issue() from the store or the checkpoint: FP8 codes and scales into the slot
 * (octet-tiled through staging when the slots are), or quantised into an int4 slot. */
int issue_reads(Glm53fCache *c, Impl *m, int slot, int layer, int expert, hipStream_t s, int64_t *nread)
{
    Glm53fExpertQ h;
    memset(&h, 0, sizeof h);
    int rc = store_view(m, layer, expert, &h);
    while (rc == G53H_CKPT_BUSY && !m->inflight.empty()) {     /* staging full: wait for a copy */
        if (hipEventSynchronize(m->inflight.front().ev) != hipSuccess) return 0;
        poll(c, m);
        rc = store_view(m, layer, expert, &h);
    }
    if (rc != 0) return 0;
    const Glm53fMat *mats[3] = {&h.gate, &h.up, &h.down};
    for (int i = 0; i < 3; i++)
        if (!same_mat(*mats[i], m->geo, i)) {
            fprintf(stderr, "glm53f_cache: L%d expert %d does not have the slot's shape\n", layer, expert);
            store_done(m, layer, expert);
            return 0;
        }
    uint8_t *base = m->arena + (size_t)slot * (size_t)c->slot_bytes;
    table_clear(c, m, slot);
    if (m->used[slot] >= 0) {
        if (hipStreamWaitEvent(s, m->used_ev[m->used[slot]], 0) != hipSuccess) return 0;
        unuse(m, slot);
    }
    if (m->landed_ok[slot] && hipStreamWaitEvent(s, m->landed[slot], 0) != hipSuccess) return 0;
    uint8_t *stage = s == m->prefetch ? m->stage_prefetch : m->stage_demand;
    for (int i = 0; m->i4 && i < 3; i++) {
        /* FP8 codes and scales into staging, then the quantiser into the slot */
        const size_t sc_off = al(m->geo.fbytes[i], 256);
        G53hMat f;
        memset(&f, 0, sizeof f);
        f.w = stage; f.s = (const float *)(stage + sc_off);
        f.rows = m->geo.rows[i]; f.cols = m->geo.cols[i]; f.br = m->geo.br[i]; f.bc = m->geo.bc[i];
        f.scols = m->geo.scols[i];
        /* int4 modes 2, 3: the levels (mode 3: and the steps) into staging after the FP8 bytes,
         * then tiled into the slot */
        uint8_t *lv = (m->i4t || m->i4m) ? stage + m->stage_lv : base + m->geo.off[i];
        float *sl = (float *)(m->i4m ? stage + m->stage_st : base + m->geo.off[3 + i]);
        if (hipMemcpyAsync(stage, mats[i]->w, m->geo.fbytes[i], hipMemcpyHostToDevice, s) != hipSuccess ||
            hipMemcpyAsync(stage + sc_off, mats[i]->s, m->geo.fbytes[3 + i], hipMemcpyHostToDevice, s) !=
                hipSuccess ||
            g53h_i4_from_f8_on(lv, sl, &f, s) ||
            (m->i4t && g53h_tile_i4_on(base + m->geo.off[i], lv, m->geo.rows[i], m->geo.cols[i], 0, s)) ||
            (m->i4m && g53h_mtile_i4_on(base + m->geo.off[i], (float *)(base + m->geo.off[3 + i]), lv, sl,
                                        m->geo.rows[i], m->geo.cols[i], 0, s)))
            return 0;
        *nread += (int64_t)(m->geo.fbytes[i] + m->geo.fbytes[3 + i]);
    }
    for (int i = 0; !m->i4 && i < 3; i++) {
        if (m->tiled) {
            if (hipMemcpyAsync(stage, mats[i]->w, m->geo.bytes[i], hipMemcpyHostToDevice, s) != hipSuccess ||
                (m->mt ? g53h_mtile_f8_on(base + m->geo.off[i], stage, m->geo.rows[i], m->geo.cols[i], 0, s)
                       : g53h_tile_f8_on(base + m->geo.off[i], stage, m->geo.rows[i], m->geo.cols[i], s)))
                return 0;
        } else if (hipMemcpyAsync(base + m->geo.off[i], mats[i]->w, m->geo.bytes[i], hipMemcpyHostToDevice, s) !=
                   hipSuccess) {
            return 0;
        }
        if (hipMemcpyAsync(base + m->geo.off[3 + i], mats[i]->s, m->geo.bytes[3 + i], hipMemcpyHostToDevice, s) !=
            hipSuccess)
            return 0;
        *nread += (int64_t)(m->geo.bytes[i] + m->geo.bytes[3 + i]);
    }
    return 1;
}

/* Start queued prefetch reads while fewer than n_io are in flight. */
void pump(Glm53fCache *c, Impl *m)
{
    int busy = 0;
    for (const Copy &cp : m->inflight) busy += cp.background;
    while (busy < c->n_io) {
        const int32_t key = g53_lru_pop(&m->lru);
        if (key < 0) break;
        const int slot = g53_lru_reserve(&m->lru, key);
        if (slot < 0) continue;                       /* cache saturated: skip this hint */
        int64_t nread = 0;
        const int ok = issue(c, m, slot, key / c->n_experts, key % c->n_experts, m->prefetch, 1, &nread);
        g53_lru_land(&m->lru, key, slot, ok, 1);
        if (ok) { m->lru.bg_reads++; c->bg_bytes += (uint64_t)nread; busy++; }
    }
}

void view_of(const Glm53fCache *c, const Impl *m, int slot, Glm53fExpertQ *q)
{
    uint8_t *base = m->arena + (size_t)slot * (size_t)c->slot_bytes;
    Glm53fMat *mats[3] = {&q->gate, &q->up, &q->down};
    for (int i = 0; i < 3; i++) {
        Glm53fMat &v = *mats[i];
        v.w = base + m->geo.off[i];
        v.s = (const float *)(base + m->geo.off[3 + i]);
        v.dt = m->i4 ? (m->i4t ? GLM53F_WI4T : m->i4m ? GLM53F_WI4M : GLM53F_WI4)
                     : (m->tiled ? (m->mt ? GLM53F_WF8M : GLM53F_WF8T) : GLM53F_WF8);
        v.rows = m->geo.rows[i]; v.cols = m->geo.cols[i];
        if (m->i4) {                                 /* glm53f_expert_i4_view's geometry */
            v.br = 1; v.bc = GLM53F_I4_GROUP; v.scols = m->geo.cols[i] / GLM53F_I4_GROUP;
        } else {
            v.br = m->geo.br[i]; v.bc = m->geo.bc[i]; v.scols = m->geo.scols[i];
        }
    }
}

int cache_get(Glm53fExpertSrc *self, int layer, int expert, Glm53fExpertQ *out)
{
    Glm53fCache *c = (Glm53fCache *)self;
    Impl *m = impl_of(c);
    if (layer < 0 || layer >= c->n_layers || expert < 0 || expert >= c->n_experts) {
        fprintf(stderr, "glm53f_cache: out of range L%d expert %d\n", layer, expert);
        return -1;
    }
    const int32_t key = layer * c->n_experts + expert;
    const double t0 = now_s();
    std::lock_guard<std::mutex> g(m->mu);
    poll(c, m);
    if (m->cur_used >= 0 && m->used_refs[m->cur_used] == 0) m->used_free.push_back(m->cur_used);
    m->cur_used = -1;                 /* kernels launched after this use a later release event */
    int slot = g53_lru_hit(&m->lru, key);
    if (slot < 0) {
        m->lru.misses++;
        const int s = g53_lru_reserve(&m->lru, key);
        if (s < 0) {          /* every slot pinned: the caller holds more than the cache can */
            fprintf(stderr, "glm53f_cache: all %d slots are pinned; cannot read L%d expert %d\n", c->nslot, layer,
                    expert);
            m->lru.misses--;
            c->load_seconds += now_s() - t0;
            return -1;
        }
        int64_t nread = 0;
        const int ok = issue(c, m, s, layer, expert, m->demand, 0, &nread);
        g53_lru_land(&m->lru, key, s, ok, 0);
        if (!ok) {
            fprintf(stderr, "glm53f_cache: short load of L%d expert %d\n", layer, expert);
            sync_stats(c, m);
            c->load_seconds += now_s() - t0;
            return -1;
        }
        c->bytes_read += (uint64_t)nread;
        slot = g53_lru_hit(&m->lru, key);
        m->lru.hits--;                                /* the read, not a hit */
    }
    /* kernels on the compute stream after this point see the slot's bytes */
    if (m->landed_ok[slot] && hipStreamWaitEvent(g53h_stream(), m->landed[slot], 0) != hipSuccess) {
        g53_lru_release(&m->lru, key);
        return -1;
    }
    view_of(c, m, slot, out);
    pump(c, m);
    sync_stats(c, m);
    c->load_seconds += now_s() - t0;
    return 0;
}

void cache_release(Glm53fExpertSrc *self, int layer, int expert)
{
    Glm53fCache *c = (Glm53fCache *)self;
    Impl *m = impl_of(c);
    if (layer < 0 || layer >= c->n_layers || expert < 0 || expert >= c->n_experts) return;
    const int32_t key = layer * c->n_experts + expert;
    std::lock_guard<std::mutex> g(m->mu);
    const int slot = m->lru.slot_of[key];
    if (slot >= 0 && m->lru.pins[slot] > 0 && g53h_quiet()) {
        /* every kernel launched so far has completed: a refill of the slot waits for nothing */
        unuse(m, slot);
        g53_lru_release(&m->lru, key);
    } else if (slot >= 0 && m->lru.pins[slot] > 0) {
        /* one event for all releases between two get() calls: the caller launched the kernels
         * that read these slots before releasing any of them */
        if (m->cur_used < 0) {
            int u;
            if (!m->used_free.empty()) { u = m->used_free.back(); m->used_free.pop_back(); }
            else {
                hipEvent_t e;
                if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) return;
                u = (int)m->used_ev.size();
                m->used_ev.push_back(e);
                m->used_refs.push_back(0);
            }
            if (hipEventRecord(m->used_ev[u], g53h_stream()) != hipSuccess) return;
            m->cur_used = u;
        }
        unuse(m, slot);
        m->used[slot] = m->cur_used;
        m->used_refs[m->cur_used]++;
        g53_lru_release(&m->lru, key);
    }
    poll(c, m);
    pump(c, m);
    sync_stats(c, m);
}

int cache_getmany(Glm53fExpertSrc *self, int layer, const int *ids, int n)
{
    Glm53fCache *c = (Glm53fCache *)self;
    Impl *m = impl_of(c);
    const double t0 = now_s();
    std::lock_guard<std::mutex> g(m->mu);
    poll(c, m);
    int keys[GLM53F_MAX_TOPK], slots[GLM53F_MAX_TOPK], nw = 0;
    for (int i = 0; i < n && nw < GLM53F_MAX_TOPK; i++) {
        const int e = ids[i];
        if (e < 0 || e >= c->n_experts || layer < 0 || layer >= c->n_layers) continue;
        const int32_t key = layer * c->n_experts + e;
        if (m->lru.slot_of[key] >= 0 || m->lru.inflight_of[key] >= 0) continue;
        const int s = g53_lru_reserve(&m->lru, key);
        if (s < 0) break;
        keys[nw] = key; slots[nw] = s; nw++;
    }
    int ok_n = 0;
    for (int k = 0; k < nw; k++) {
        int64_t nread = 0;
        const int ok = issue(c, m, slots[k], layer, keys[k] % c->n_experts, m->demand, 0, &nread);
        g53_lru_land(&m->lru, keys[k], slots[k], ok, 0);
        if (!ok) {
            fprintf(stderr, "glm53f_cache: short prefetch of L%d expert %d; slot left empty\n", layer,
                    keys[k] % c->n_experts);
            continue;
        }
        c->bytes_read += (uint64_t)nread;
        m->lru.prefetch_reads++;
        ok_n++;
    }
    sync_stats(c, m);
    c->load_seconds += now_s() - t0;
    return ok_n;
}

void cache_hint(Glm53fExpertSrc *self, int layer, const int *ids, int n)
{
    Glm53fCache *c = (Glm53fCache *)self;
    Impl *m = impl_of(c);
    if (c->n_io <= 0 || layer < 0 || layer >= c->n_layers) return;
    std::lock_guard<std::mutex> g(m->mu);
    g53_lru_hint(&m->lru, layer, ids, n);
    poll(c, m);
    pump(c, m);
    sync_stats(c, m);
}

} /* namespace */

extern "C" int g53h_cache_is(const Glm53fExpertSrc *src) { return src && src->get == cache_get; }

extern "C" int g53h_cache_slot_kind(const Glm53fExpertSrc *src)
{
    if (!g53h_cache_is(src)) return 0;
    const Impl *m = impl_of((const Glm53fCache *)src);
    return !m ? 0 : m->tiled ? (m->mt ? 2 : 1) : m->i4t ? 3 : m->i4m ? 4 : 0;
}

extern "C" int g53h_cache_layer_table(Glm53fExpertSrc *src, int layer, const G53hExpert **table_d,
                                      const G53hExpert **table_h)
{
    if (!g53h_cache_is(src)) return -1;
    Glm53fCache *c = (Glm53fCache *)src;
    Impl *m = impl_of(c);
    if (!m || !m->tab_h || layer < 0 || layer >= c->n_layers) return -1;
    std::lock_guard<std::mutex> g(m->mu);
    poll(c, m);
    if (m->pend[layer] > 0) return m->pend[layer];
    const size_t nb = (size_t)c->n_experts * sizeof(G53hExpert);
    G53hExpert *h = m->tab_h + (size_t)layer * c->n_experts, *d = m->tab_d + (size_t)layer * c->n_experts;
    if (m->tab_dirty[layer]) {
        if (hipMemcpyAsync(d, h, nb, hipMemcpyHostToDevice, g53h_stream()) != hipSuccess) return -1;
        m->tab_dirty[layer] = 0;
    }
    *table_d = d;
    *table_h = h;
    return 0;
}

/* Common set-up once the store is known (m->store or m->ckpt). */
static int cache_setup(Glm53fCache *c, Impl *m, const Glm53fCfg *cfg, int64_t budget_bytes, int n_io, int i4)
{
    c->cfg = cfg;
    c->n_layers = cfg->n_layers + 1;       /* the MTP layer streams experts the same way */
    c->n_experts = cfg->n_experts;
    c->hint_floor = c->last_hint = -1;
    int probe = -1;
    for (int L = 0; L < cfg->n_layers && L < GLM53F_MAX_LAYERS; L++)
        if (!cfg->is_dense[L]) { probe = L; break; }
    if (probe < 0) { delete m; return 0; }  /* no MoE layers: nothing to cache */
    Glm53fExpertQ h;
    memset(&h, 0, sizeof h);
    if (store_view(m, probe, 0, &h) != 0) {
        fprintf(stderr, "glm53f_cache: cannot resolve expert 0 of layer %d\n", probe);
        delete m;
        return -1;
    }
    store_done(m, probe, 0);
    const Glm53fMat *mats[3] = {&h.gate, &h.up, &h.down};
    size_t off = 0;
    for (int i = 0; i < 3; i++) {
        if (mats[i]->dt != GLM53F_WF8) {
            fprintf(stderr, "glm53f_cache: expert matrices must be FP8\n");
            delete m;
            return -1;
        }
        m->geo.rows[i] = mats[i]->rows; m->geo.cols[i] = mats[i]->cols;
        m->geo.br[i] = mats[i]->br; m->geo.bc[i] = mats[i]->bc; m->geo.scols[i] = mats[i]->scols;
        m->geo.off[i] = off;
        m->geo.bytes[i] = (size_t)mats[i]->rows * (size_t)mats[i]->cols;
        off = al(off + m->geo.bytes[i], 256);
    }
    for (int i = 0; i < 3; i++) {
        m->geo.off[3 + i] = off;
        m->geo.bytes[3 + i] = scale_bytes(*mats[i]);
        off = al(off + m->geo.bytes[3 + i], 256);
    }
    c->slot_bytes = (int64_t)al(off, 4096);
    m->i4 = i4 != 0;
    c->i4 = m->i4 ? 1 : 0;
    if (m->i4) {
        for (int i = 0; i < 3; i++)
            if (m->geo.cols[i] % GLM53F_I4_GROUP) {
                fprintf(stderr, "glm53f_cache: int4 slots need columns a multiple of %d\n", GLM53F_I4_GROUP);
                delete m;
                return -1;
            }
        /* the reference's int4 slot (src/io/glm53f_load.c:141-163): per matrix the levels, then
         * the steps, each 64-byte aligned; the slot rounded up to 4096 bytes */
        size_t o = 0;
        for (int i = 0; i < 3; i++) {
            m->geo.fbytes[i] = m->geo.bytes[i];
            m->geo.fbytes[3 + i] = m->geo.bytes[3 + i];
            o = al(o, 64);
            m->geo.off[i] = o;
            m->geo.bytes[i] = (size_t)m->geo.rows[i] * (size_t)(m->geo.cols[i] / 2);
            o += m->geo.bytes[i];
            o = al(o, 64);
            m->geo.off[3 + i] = o;
            m->geo.bytes[3 + i] = (size_t)m->geo.rows[i] * (size_t)(m->geo.cols[i] / GLM53F_I4_GROUP) * 4;
            o += m->geo.bytes[3 + i];
        }
        c->slot_bytes = (int64_t)al(o, 4096);
    }
    /* slots octet-tiled at the shapes the one-launch tiled decode reads (hidden 4096, inter
     * 2048, 128 x 128 blocks), row-major otherwise or with GLM53F_CACHE_ROWMAJOR set */
    m->tiled = !getenv("GLM53F_CACHE_ROWMAJOR") && m->geo.rows[0] == 2048 && m->geo.cols[0] == 4096 &&
               m->geo.rows[1] == 2048 && m->geo.cols[1] == 4096 && m->geo.rows[2] == 4096 && m->geo.cols[2] == 2048;
    for (int i = 0; i < 3; i++) m->tiled = m->tiled && m->geo.br[i] == 128 && m->geo.bc[i] == 128;
    /* int4 mode 2 at the shapes the octet test above accepts (their rows are multiples of 8 and
     * columns of 256, as the int4 tiling needs) */
    m->i4t = m->i4 && i4 == 2 && m->tiled;
    m->i4m = m->i4 && i4 == 3 && m->tiled;      /* int4 mode 3: the same shapes, MFMA-tiled */
    if (m->i4) m->tiled = false;
    /* FP8 slots MFMA-tiled (the FP8 matrix-core decode) at the same shapes, when asked */
    {
        const char *e = getenv("GLM53F_CACHE_MFMA");
        m->mt = m->tiled && e && atoi(e) != 0;
    }
    if (m->i4t) c->i4 = 2;
    if (m->i4m) c->i4 = 3;
    c->nslot = (int)(budget_bytes / c->slot_bytes);
    if (c->nslot < cfg->topk + 1) {
        fprintf(stderr, "glm53f_cache: budget %.2f GB gives %d slots of %.2f MB; top-%d needs at least %d\n",
                (double)budget_bytes / 1e9, c->nslot, (double)c->slot_bytes / 1e6, cfg->topk, cfg->topk + 1);
        delete m;
        return -1;
    }
    if (g53_lru_init(&m->lru, c->n_layers, c->n_experts, c->nslot, 64 * 4 * GLM53F_MAX_TOPK) != 0) {
        delete m;
        return -1;
    }
    m->arena = (uint8_t *)g53h_alloc((size_t)c->nslot * (size_t)c->slot_bytes);
    if (!m->arena) {
        fprintf(stderr, "glm53f_cache: cannot allocate a %.2f GB arena in HBM\n",
                (double)c->nslot * (double)c->slot_bytes / 1e9);
        g53_lru_free(&m->lru);
        delete m;
        return -1;
    }
    m->landed.resize(c->nslot);
    m->landed_ok.assign(c->nslot, 0);
    m->gen.assign(c->nslot, 0);
    m->used.assign(c->nslot, -1);
    bool ok = true;
    for (int i = 0; i < c->nslot && ok; i++)
        ok = hipEventCreateWithFlags(&m->landed[i], hipEventDisableTiming) == hipSuccess;
    m->demand = g53h_copy_stream();
    ok = ok && hipStreamCreateWithFlags(&m->prefetch, hipStreamNonBlocking) == hipSuccess;
    if (ok && (m->tiled || m->i4)) {
        size_t sb = 0;                               /* the largest matrix (with its scales) */
        size_t lb = 0;                               /* the largest matrix's int4 levels */
        size_t stb = 0;                              /* and its steps */
        for (int i = 0; i < 3; i++) {
            const size_t need = m->i4 ? al(m->geo.fbytes[i], 256) + m->geo.fbytes[3 + i] : m->geo.bytes[i];
            if (need > sb) sb = need;
            if (m->i4 && m->geo.bytes[i] > lb) lb = m->geo.bytes[i];
            if (m->i4 && m->geo.bytes[3 + i] > stb) stb = m->geo.bytes[3 + i];
        }
        if (m->i4t || m->i4m) {
            m->stage_lv = al(sb, 256);
            sb = m->stage_lv + lb;
        }
        if (m->i4m) {
            m->stage_st = al(sb, 256);
            sb = m->stage_st + stb;
        }
        m->stage_demand = (uint8_t *)g53h_alloc(sb);
        m->stage_prefetch = (uint8_t *)g53h_alloc(sb);
        ok = m->stage_demand && m->stage_prefetch;
    }
    if (ok && (m->tiled || m->i4t || m->i4m)) {
        const size_t tb = (size_t)c->n_layers * (size_t)c->n_experts * sizeof(G53hExpert);
        m->tab_h = (G53hExpert *)g53h_host_alloc(tb);
        m->tab_d = (G53hExpert *)g53h_alloc(tb);
        ok = m->tab_h && m->tab_d && !g53h_memset(m->tab_d, 0, tb);
        if (m->tab_h) memset(m->tab_h, 0, tb);
        m->tab_dirty.assign(c->n_layers, 0);
        m->tab_key.assign(c->nslot, -1);
        m->pend.assign(c->n_layers, 0);
    }
    c->stage = (unsigned char **)(void *)m;
    if (!ok) {
        fprintf(stderr, "glm53f_cache: cannot create the copy events and streams\n");
        glm53f_cache_free(c);
        return -1;
    }
    c->arena = m->arena;
    c->slot_of = m->lru.slot_of;
    c->inflight_of = m->lru.inflight_of;
    c->key_of = m->lru.key_of;
    c->pins = m->lru.pins;
    c->prefetched = m->lru.prefetched;
    c->used_at = m->lru.used_at;
    c->queued = m->lru.queued;
    c->qcap = m->lru.qcap;
    c->n_io = n_io > 0 ? n_io : 0;
    c->src.get = cache_get;
    c->src.release = cache_release;
    c->src.getmany = cache_getmany;
    c->src.hint = cache_hint;
    c->src.ctx = c;
    sync_stats(c, m);
    return 0;
}

extern "C" int glm53f_cache_init(Glm53fCache *c, const Glm53fSt *st, const Glm53fCfg *cfg, int64_t budget_bytes,
                                 int n_io, int i4)
{
    memset(c, 0, sizeof *c);
    if (!st || !cfg) return -1;
    if (g53h_ready()) {
        fprintf(stderr, "glm53f_cache: %s\n", g53h_error());
        return -1;
    }
    Impl *m = new Impl();
    /* staging: one buffer per prefetch read in flight, plus room for demand reads */
    m->ckpt = g53h_ckpt_new(st, cfg, cfg->n_layers + 1, (n_io > 0 ? n_io : 0) + 4);
    if (!m->ckpt) {
        fprintf(stderr, "glm53f_cache: cannot index the checkpoint or allocate pinned staging\n");
        delete m;
        return -1;
    }
    c->st = st;
    return cache_setup(c, m, cfg, budget_bytes, n_io, i4);
}

extern "C" int g53h_cache_init_store(Glm53fCache *c, const G53hStore *store, const Glm53fCfg *cfg,
                                     int64_t budget_bytes, int n_io, int i4)
{
    memset(c, 0, sizeof *c);
    if (!store || !store->view || !cfg) return -1;
    if (g53h_ready()) {
        fprintf(stderr, "glm53f_cache: %s\n", g53h_error());
        return -1;
    }
    Impl *m = new Impl();
    m->store = store;
    return cache_setup(c, m, cfg, budget_bytes, n_io, i4);
}

extern "C" int glm53f_cache_sync(Glm53fCache *c)
{
    Impl *m = impl_of(c);
    if (!m) return 0;
    std::lock_guard<std::mutex> g(m->mu);
    if (hipStreamSynchronize(m->demand) != hipSuccess || hipStreamSynchronize(m->prefetch) != hipSuccess) return -1;
    poll(c, m);
    return 0;
}

extern "C" void glm53f_cache_free(Glm53fCache *c)
{
    Impl *m = impl_of(c);
    if (m) {
        (void)hipDeviceSynchronize();
        poll(c, m);
        for (hipEvent_t e : m->landed) if (e) (void)hipEventDestroy(e);
        for (hipEvent_t e : m->used_ev) (void)hipEventDestroy(e);
        for (hipEvent_t e : m->pool) (void)hipEventDestroy(e);
        for (Copy &cp : m->inflight) (void)hipEventDestroy(cp.ev);
        if (m->prefetch) (void)hipStreamDestroy(m->prefetch);
        if (m->arena) g53h_free(m->arena);
        g53h_free(m->stage_demand);
        g53h_free(m->stage_prefetch);
        g53h_free(m->tab_d);
        g53h_host_free(m->tab_h);
        g53_lru_free(&m->lru);
        delete m;
    }
    memset(c, 0, sizeof *c);
}

extern "C" void glm53f_cache_reset_stats(Glm53fCache *c)
{
    Impl *m = impl_of(c);
    if (!m) return;
    std::lock_guard<std::mutex> g(m->mu);
    m->lru.hits = m->lru.misses = m->lru.evictions = m->lru.prefetch_reads = 0;
    m->lru.bg_reads = m->lru.bg_used = 0;
    c->bytes_read = c->bg_bytes = 0;
    c->load_seconds = 0.0;
    sync_stats(c, m);
}

extern "C" void glm53f_cache_report(const Glm53fCache *c, const char *label)
{
    const Impl *m = impl_of(c);
    if (!m || glm53f_quiet) return;
    int resident = 0;
    for (int i = 0; i < c->nslot; i++) if (m->lru.key_of[i] >= 0) resident++;
    const uint64_t n = c->hits + c->misses;
    const uint64_t served = c->hits > c->prefetch_reads ? c->hits - c->prefetch_reads : 0;
    printf("expert cache [%s]\n", label ? label : "");
    printf("  slots          : %d x %.2f MB = %.2f GB of HBM (%d resident), %d prefetch reads in flight\n",
           c->nslot, (double)c->slot_bytes / 1e6, (double)c->nslot * c->slot_bytes / 1e9, resident, c->n_io);
    printf("  requests       : %llu, resident when requested: %llu (%.1f%%)\n", (unsigned long long)n,
           (unsigned long long)served, n ? 100.0 * served / n : 0.0);
    printf("  foreground     : %.2f GB copied to HBM, %.3f s in get/getmany, %llu evictions\n",
           (double)c->bytes_read / 1e9, c->load_seconds, (unsigned long long)c->evictions);
    if (c->n_io)
        printf("  prefetch       : %llu experts read ahead (%.2f GB), %llu of them used\n",
               (unsigned long long)c->bg_reads, (double)c->bg_bytes / 1e9, (unsigned long long)c->bg_used);
}

/* ------------------------------------------------------- synthetic host store ---- */
namespace {

struct SynthStore {
    int hidden, inter, n_layers, n_experts, n_pool;
    uint8_t *pinned;                 /* n_pool experts: codes g, u, d, scales g, u, d */
    size_t per, off[6];
    float *kscales = nullptr;        /* optional: per key, scales g, u, d back to back  */
    size_t kper = 0, koff[3] = {0, 0, 0};
};

int synth_view(const G53hStore *st, int layer, int expert, Glm53fExpertQ *h)
{
    const SynthStore *s = (const SynthStore *)st->ctx;
    if (layer < 0 || layer >= s->n_layers || expert < 0 || expert >= s->n_experts) return -1;
    const long key = (long)layer * s->n_experts + expert;
    const uint8_t *b = s->pinned + (size_t)(key % s->n_pool) * s->per;
    const int rows[3] = {s->inter, s->inter, s->hidden}, cols[3] = {s->hidden, s->hidden, s->inter};
    Glm53fMat *mats[3] = {&h->gate, &h->up, &h->down};
    for (int i = 0; i < 3; i++) {
        Glm53fMat &m = *mats[i];
        m.w = b + s->off[i];
        m.s = s->kscales ? s->kscales + (size_t)key * s->kper + s->koff[i] : (const float *)(b + s->off[3 + i]);
        m.dt = GLM53F_WF8;
        m.rows = rows[i]; m.cols = cols[i];
        m.br = 128; m.bc = 128;
        m.scols = (cols[i] + 127) / 128;
    }
    return 0;
}

} /* namespace */

extern "C" int g53h_store_synth_init(G53hStore *st, int hidden, int inter, int n_layers, int n_experts, int n_pool,
                                     uint64_t seed, float sigma)
{
    memset(st, 0, sizeof *st);
    if (hidden <= 0 || inter <= 0 || n_layers <= 0 || n_experts <= 0 || n_pool <= 0) return -1;
    if (g53h_ready()) return -1;
    SynthStore *s = new SynthStore();
    s->hidden = hidden; s->inter = inter; s->n_layers = n_layers; s->n_experts = n_experts; s->n_pool = n_pool;
    const int rows[3] = {inter, inter, hidden}, cols[3] = {hidden, hidden, inter};
    size_t off = 0;
    for (int i = 0; i < 3; i++) { s->off[i] = off; off = al(off + (size_t)rows[i] * cols[i], 256); }
    for (int i = 0; i < 3; i++) {
        s->off[3 + i] = off;
        off = al(off + (size_t)((rows[i] + 127) / 128) * ((cols[i] + 127) / 128) * 4, 256);
    }
    s->per = al(off, 4096);
    s->pinned = (uint8_t *)g53h_host_alloc(s->per * (size_t)n_pool);
    uint8_t *dev = (uint8_t *)g53h_alloc(s->per);
    if (!s->pinned || !dev) {
        if (s->pinned) g53h_host_free(s->pinned);
        if (dev) g53h_free(dev);
        delete s;
        return g53h_fail("g53h_store_synth_init: cannot allocate %zu bytes of pinned host memory", s->per * (size_t)n_pool);
    }
    /* pool entry p is expert p of the synthetic layer 0: the streams of glm53h.synth */
    for (int p = 0; p < n_pool; p++) {
        for (int i = 0; i < 3; i++) {
            const uint64_t strm = (4ull << 32) | (uint64_t)(p * 3 + i);
            if (g53h_synth_f8(dev + s->off[i], (float *)(dev + s->off[3 + i]), rows[i], cols[i], 128, 128, seed, strm,
                              sigma))
                goto fail;
        }
        if (g53h_sync() || g53h_d2h(s->pinned + (size_t)p * s->per, dev, s->per)) goto fail;
    }
    g53h_free(dev);
    st->view = synth_view;
    st->done = nullptr;
    st->ctx = s;
    return 0;
fail:
    g53h_free(dev);
    g53h_host_free(s->pinned);
    delete s;
    return -1;
}

extern "C" int g53h_store_synth_key_scales(G53hStore *st)
{
    SynthStore *s = st ? (SynthStore *)st->ctx : nullptr;
    if (!s || st->view != synth_view) return g53h_fail("g53h_store_synth_key_scales: not a synthetic store");
    if (s->kscales) return 0;
    const int rows[3] = {s->inter, s->inter, s->hidden}, cols[3] = {s->hidden, s->hidden, s->inter};
    size_t n[3], tot = 0;
    for (int i = 0; i < 3; i++) {
        n[i] = (size_t)((rows[i] + 127) / 128) * ((cols[i] + 127) / 128);
        s->koff[i] = tot;
        tot += n[i];
    }
    const size_t keys = (size_t)s->n_layers * s->n_experts;
    float *k = (float *)g53h_host_alloc(keys * tot * sizeof(float));
    if (!k) return g53h_fail("g53h_store_synth_key_scales: cannot allocate %zu bytes of pinned memory", keys * tot * 4);
    for (size_t key = 0; key < keys; key++) {
        const uint8_t *b = s->pinned + (key % (size_t)s->n_pool) * s->per;
        const float f = 1.0f + (float)(key + 1) * (1.0f / 16384.0f);
        for (int i = 0; i < 3; i++) {
            const float *src = (const float *)(b + s->off[3 + i]);
            for (size_t j = 0; j < n[i]; j++) k[key * tot + s->koff[i] + j] = src[j] * f;
        }
    }
    s->kscales = k;
    s->kper = tot;
    return 0;
}

extern "C" void g53h_store_synth_free(G53hStore *st)
{
    SynthStore *s = (SynthStore *)st->ctx;
    if (s) {
        if (s->kscales) g53h_host_free(s->kscales);
        g53h_host_free(s->pinned);
        delete s;
    }
    memset(st, 0, sizeof *st);
}
