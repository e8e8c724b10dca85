/* g53h_lru.c - see g53h_lru.h. */
#include "g53h_lru.h"

#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------- EMPTY bitmap ---- */
static void empty_set(G53hLru *c, int s)
{
    c->empty_w[s >> 6] |= 1ull << (s & 63);
    c->empty_s[s >> 12] |= 1ull << ((s >> 6) & 63);
}

static void empty_clear(G53hLru *c, int s)
{
    uint64_t *w = &c->empty_w[s >> 6];
    *w &= ~(1ull << (s & 63));
    if (!*w) c->empty_s[s >> 12] &= ~(1ull << ((s >> 6) & 63));
}

static int empty_first(const G53hLru *c)
{
    const int nsum = (c->nslot + 4095) >> 12;
    for (int i = 0; i < nsum; i++) {
        if (!c->empty_s[i]) continue;
        const int w = (i << 6) + __builtin_ctzll(c->empty_s[i]);
        return (w << 6) + __builtin_ctzll(c->empty_w[w]);
    }
    return -1;
}

/* ------------------------------------------------- evictable slots: min-heap ---- */
static int heap_less(const G53hLru *c, int a, int b) { return c->used_at[a] < c->used_at[b]; }

static void heap_place(G53hLru *c, int at, int s)
{
    c->heap[at] = s;
    c->heap_at[s] = at;
}

static void heap_up(G53hLru *c, int at)
{
    const int s = c->heap[at];
    while (at > 0) {
        const int up = (at - 1) >> 1;
        if (!heap_less(c, s, c->heap[up])) break;
        heap_place(c, at, c->heap[up]);
        at = up;
    }
    heap_place(c, at, s);
}

static void heap_down(G53hLru *c, int at)
{
    const int s = c->heap[at];
    for (;;) {
        int kid = 2 * at + 1;
        if (kid >= c->heap_n) break;
        if (kid + 1 < c->heap_n && heap_less(c, c->heap[kid + 1], c->heap[kid])) kid++;
        if (!heap_less(c, c->heap[kid], s)) break;
        heap_place(c, at, c->heap[kid]);
        at = kid;
    }
    heap_place(c, at, s);
}

static void heap_add(G53hLru *c, int s)
{
    heap_place(c, c->heap_n++, s);
    heap_up(c, c->heap_n - 1);
}

static void heap_del(G53hLru *c, int s)
{
    const int at = c->heap_at[s];
    if (at < 0) return;
    c->heap_at[s] = -1;
    const int last = c->heap[--c->heap_n];
    if (at == c->heap_n) return;
    heap_place(c, at, last);
    heap_up(c, at);
    heap_down(c, c->heap_at[last]);
}

/* ---------------------------------------------------------------- lifecycle ---- */
int g53_lru_init(G53hLru *c, int n_layers, int n_experts, int nslot, int qcap)
{
    memset(c, 0, sizeof *c);
    if (n_layers < 1 || n_experts < 1 || nslot < 1 || qcap < 1) return -1;
    const size_t nkey = (size_t)n_layers * (size_t)n_experts;
    const size_t nw = ((size_t)nslot + 63) >> 6, ns = ((size_t)nslot + 4095) >> 12;
    c->n_layers = n_layers;
    c->n_experts = n_experts;
    c->nslot = nslot;
    c->qcap = qcap;
    c->slot_of = (int32_t *)malloc(nkey * sizeof(int32_t));
    c->inflight_of = (int32_t *)malloc(nkey * sizeof(int32_t));
    c->queued = (unsigned char *)calloc(nkey, 1);
    c->key_of = (int32_t *)malloc((size_t)nslot * sizeof(int32_t));
    c->pins = (int32_t *)calloc((size_t)nslot, sizeof(int32_t));
    c->prefetched = (unsigned char *)calloc((size_t)nslot, 1);
    c->used_at = (uint64_t *)calloc((size_t)nslot, sizeof(uint64_t));
    c->empty_w = (uint64_t *)calloc(nw, sizeof(uint64_t));
    c->empty_s = (uint64_t *)calloc(ns, sizeof(uint64_t));
    c->heap = (int32_t *)malloc((size_t)nslot * sizeof(int32_t));
    c->heap_at = (int32_t *)malloc((size_t)nslot * sizeof(int32_t));
    c->q_key = (int32_t *)malloc((size_t)qcap * sizeof(int32_t));
    c->q_next = (int32_t *)malloc((size_t)qcap * sizeof(int32_t));
    c->q_head = (int32_t *)malloc((size_t)n_layers * sizeof(int32_t));
    c->q_tail = (int32_t *)malloc((size_t)n_layers * sizeof(int32_t));
    c->mark = (int32_t *)calloc((size_t)n_experts, sizeof(int32_t));
    if (!c->slot_of || !c->inflight_of || !c->queued || !c->key_of || !c->pins || !c->prefetched ||
        !c->used_at || !c->empty_w || !c->empty_s || !c->heap || !c->heap_at || !c->q_key || !c->q_next ||
        !c->q_head || !c->q_tail || !c->mark) {
        g53_lru_free(c);
        return -1;
    }
    for (size_t i = 0; i < nkey; i++) { c->slot_of[i] = -1; c->inflight_of[i] = -1; }
    for (int s = 0; s < nslot; s++) {
        c->key_of[s] = G53_LRU_EMPTY;
        c->heap_at[s] = -1;
        empty_set(c, s);
    }
    for (int i = 0; i < qcap; i++) c->q_next[i] = i + 1 < qcap ? i + 1 : -1;
    c->q_free = 0;
    for (int L = 0; L < n_layers; L++) c->q_head[L] = c->q_tail[L] = -1;
    c->last_hint = -1;
    return 0;
}

void g53_lru_free(G53hLru *c)
{
    free(c->slot_of); free(c->inflight_of); free(c->queued); free(c->key_of); free(c->pins);
    free(c->prefetched); free(c->used_at); free(c->empty_w); free(c->empty_s); free(c->heap);
    free(c->heap_at); free(c->q_key); free(c->q_next); free(c->q_head); free(c->q_tail); free(c->mark);
    memset(c, 0, sizeof *c);
}

/* ------------------------------------------------------------------ slots ---- */
int g53_lru_pick_victim(const G53hLru *c)
{
    const int e = empty_first(c);
    if (e >= 0) return e;
    return c->heap_n ? c->heap[0] : -1;
}

int g53_lru_reserve(G53hLru *c, int32_t key)
{
    const int s = g53_lru_pick_victim(c);
    if (s < 0) return -1;
    const int32_t old = c->key_of[s];
    if (old == G53_LRU_EMPTY) {
        empty_clear(c, s);
    } else {                                   /* a resident, unpinned slot: evict its expert */
        heap_del(c, s);
        c->slot_of[old] = -1;
        c->evictions++;
    }
    c->key_of[s] = G53_LRU_INFLIGHT;
    c->prefetched[s] = 0;
    c->inflight_of[key] = s;
    return s;
}

void g53_lru_land(G53hLru *c, int32_t key, int slot, int ok, int background)
{
    c->inflight_of[key] = -1;
    if (!ok) {
        c->key_of[slot] = G53_LRU_EMPTY;
        empty_set(c, slot);
        return;
    }
    c->key_of[slot] = key;
    c->slot_of[key] = slot;
    c->used_at[slot] = ++c->clock;
    c->prefetched[slot] = (unsigned char)(background != 0);
    if (c->pins[slot] == 0) heap_add(c, slot);
}

int g53_lru_hit(G53hLru *c, int32_t key)
{
    const int s = c->slot_of[key];
    if (s < 0) return -1;
    c->hits++;
    if (c->prefetched[s]) { c->prefetched[s] = 0; c->bg_used++; }
    if (c->pins[s]++ == 0) heap_del(c, s);      /* pinned: not evictable until released */
    c->used_at[s] = ++c->clock;
    return s;
}

void g53_lru_release(G53hLru *c, int32_t key)
{
    const int s = c->slot_of[key];
    if (s < 0 || c->pins[s] <= 0) return;
    if (--c->pins[s] == 0) heap_add(c, s);
}

/* ---------------------------------------------------------- prefetch queue ---- */
static void q_drop_layer(G53hLru *c, int L)
{
    for (int n = c->q_head[L]; n >= 0;) {
        const int nx = c->q_next[n];
        c->queued[c->q_key[n]] = 0;
        c->q_next[n] = c->q_free;
        c->q_free = n;
        c->qlen--;
        n = nx;
    }
    c->q_head[L] = c->q_tail[L] = -1;
}

/* Keep only the entries of layer L whose expert carries the current mark, in order. */
static void q_filter_layer(G53hLru *c, int L)
{
    int head = -1, tail = -1;
    for (int n = c->q_head[L]; n >= 0;) {
        const int nx = c->q_next[n];
        const int32_t key = c->q_key[n];
        if (c->mark[key % c->n_experts] == c->mark_gen) {
            c->q_next[n] = -1;
            if (tail < 0) head = n; else c->q_next[tail] = n;
            tail = n;
        } else {
            c->queued[key] = 0;
            c->q_next[n] = c->q_free;
            c->q_free = n;
            c->qlen--;
        }
        n = nx;
    }
    c->q_head[L] = head;
    c->q_tail[L] = tail;
}

static void q_append(G53hLru *c, int L, int32_t key)
{
    const int n = c->q_free;
    c->q_free = c->q_next[n];
    c->q_key[n] = key;
    c->q_next[n] = -1;
    if (c->q_tail[L] < 0) c->q_head[L] = n; else c->q_next[c->q_tail[L]] = n;
    c->q_tail[L] = n;
    c->qlen++;
    c->queued[key] = 1;
    if (L < c->q_lo) c->q_lo = L;
}

void g53_lru_hint(G53hLru *c, int layer, const int *ids, int n)
{
    if (layer < 0 || layer >= c->n_layers) return;
    /* a hint for a layer not above the previous one marks the layer now computing */
    if (layer <= c->last_hint) c->hint_floor = layer;
    c->last_hint = layer;
    for (int L = c->q_lo; L < c->hint_floor && L < c->n_layers; L++) q_drop_layer(c, L);
    if (c->q_lo < c->hint_floor) c->q_lo = c->hint_floor;
    /* the hinted layer keeps only the entries this hint lists again */
    if (++c->mark_gen == 0) {
        memset(c->mark, 0, (size_t)c->n_experts * sizeof(int32_t));
        c->mark_gen = 1;
    }
    for (int i = 0; i < n; i++)
        if (ids[i] >= 0 && ids[i] < c->n_experts) c->mark[ids[i]] = c->mark_gen;
    q_filter_layer(c, layer);
    for (int i = 0; i < n && c->qlen < c->qcap; i++) {
        const int e = ids[i];
        if (e < 0 || e >= c->n_experts) continue;
        const int32_t key = layer * c->n_experts + e;
        if (c->queued[key] || c->slot_of[key] >= 0 || c->inflight_of[key] >= 0) continue;
        q_append(c, layer, key);
    }
}

int32_t g53_lru_pop(G53hLru *c)
{
    while (c->qlen > 0) {
        while (c->q_head[c->q_lo] < 0) c->q_lo++;
        const int L = c->q_lo, n = c->q_head[L];
        const int32_t key = c->q_key[n];
        c->q_head[L] = c->q_next[n];
        if (c->q_head[L] < 0) c->q_tail[L] = -1;
        c->q_next[n] = c->q_free;
        c->q_free = n;
        c->qlen--;
        c->queued[key] = 0;
        if (c->slot_of[key] < 0 && c->inflight_of[key] < 0) return key;
    }
    return -1;
}

int g53_lru_queue(const G53hLru *c, int32_t *keys, int cap)
{
    int k = 0;
    for (int L = c->q_lo; L < c->n_layers && k < cap; L++)
        for (int n = c->q_head[L]; n >= 0 && k < cap; n = c->q_next[n]) keys[k++] = c->q_key[n];
    return k;
}

/* ----------------------------------------------------------- scripted traces ---- */
#include "glm53f_cache.h"

#define G53_LRU_QCAP (64 * 4 * GLM53F_MAX_TOPK)   /* the reference's queue capacity */

typedef struct {
    G53hLru c;
    int *out, cap, n, overflow;
} G53Trace;

static void emit(G53Trace *t, int v)
{
    if (t->n < t->cap) t->out[t->n++] = v;
    else t->overflow = 1;
}

static int valid_key(const G53hLru *c, int L, int e) { return L >= 0 && L < c->n_layers && e >= 0 && e < c->n_experts; }

/* get: a miss reads in place (the read always succeeds) and then takes the hit path */
static void op_get(G53Trace *t, int L, int e)
{
    G53hLru *c = &t->c;
    if (!valid_key(c, L, e)) { emit(t, -1); emit(t, 0); emit(t, -1); return; }
    const int32_t key = L * c->n_experts + e;
    const int resident = c->slot_of[key] >= 0;
    int s = g53_lru_hit(c, key);
    if (s < 0) {
        const int r = g53_lru_reserve(c, key);
        if (r < 0) { emit(t, -1); emit(t, resident); emit(t, -1); return; }
        c->misses++;
        g53_lru_land(c, key, r, 1, 0);
        s = g53_lru_hit(c, key);
        c->hits--;
    }
    emit(t, 0); emit(t, resident); emit(t, s);
}

/* getmany: reserve every listed expert not resident or in flight (up to GLM53F_MAX_TOPK),
 * then land them all */
static void op_getmany(G53Trace *t, int L, const int *ids, int n)
{
    G53hLru *c = &t->c;
    int32_t key[GLM53F_MAX_TOPK];
    int slot[GLM53F_MAX_TOPK], k = 0;
    for (int i = 0; i < n && k < GLM53F_MAX_TOPK; i++) {
        if (!valid_key(c, L, ids[i])) continue;
        const int32_t kk = L * c->n_experts + ids[i];
        if (c->slot_of[kk] >= 0 || c->inflight_of[kk] >= 0) continue;
        if ((slot[k] = g53_lru_reserve(c, kk)) < 0) break;
        key[k++] = kk;
    }
    for (int i = 0; i < k; i++) g53_lru_land(c, key[i], slot[i], 1, 0);
    c->prefetch_reads += (uint64_t)k;
    emit(t, k);
}

static void op_hint(G53Trace *t, int L, const int *ids, int n)
{
    G53hLru *c = &t->c;
    g53_lru_hint(c, L, ids, n);
    int32_t *q = (int32_t *)malloc((size_t)(c->qlen > 0 ? c->qlen : 1) * sizeof(int32_t));
    const int nq = q ? g53_lru_queue(c, q, c->qlen) : 0;
    emit(t, nq);
    for (int i = 0; i < nq; i++) emit(t, q[i]);
    free(q);
}

/* background reader: up to k queued hints become reads; a saturated cache skips a hint */
static void op_serve(G53Trace *t, int k)
{
    G53hLru *c = &t->c;
    int done = 0;
    while (done < k) {
        const int32_t key = g53_lru_pop(c);
        if (key < 0) break;
        const int s = g53_lru_reserve(c, key);
        if (s < 0) continue;
        g53_lru_land(c, key, s, 1, 1);
        c->bg_reads++;
        emit(t, key); emit(t, s);
        done++;
    }
    emit(t, -1);
}

int g53h_lru_trace(int n_layers, int n_experts, int nslot, const int *ops, int nops, int *out, int outcap,
                   long long *stats)
{
    G53Trace t;
    memset(&t, 0, sizeof t);
    if (g53_lru_init(&t.c, n_layers, n_experts, nslot, G53_LRU_QCAP)) return -1;
    t.out = out;
    t.cap = outcap;
    int bad = 0, i = 0;
    while (i < nops && !bad && !t.overflow) {
        switch (ops[i]) {
        case 1: op_get(&t, ops[i + 1], ops[i + 2]); i += 3; break;
        case 2:
            if (valid_key(&t.c, ops[i + 1], ops[i + 2])) g53_lru_release(&t.c, ops[i + 1] * n_experts + ops[i + 2]);
            i += 3;
            break;
        case 3: op_getmany(&t, ops[i + 1], ops + i + 3, ops[i + 2]); i += 3 + ops[i + 2]; break;
        case 4: op_hint(&t, ops[i + 1], ops + i + 3, ops[i + 2]); i += 3 + ops[i + 2]; break;
        case 5: op_serve(&t, ops[i + 1]); i += 2; break;
        default: bad = 1;
        }
    }
    if (stats) {
        const G53hLru *c = &t.c;
        stats[0] = (long long)c->hits; stats[1] = (long long)c->misses; stats[2] = (long long)c->evictions;
        stats[3] = (long long)c->prefetch_reads; stats[4] = (long long)c->bg_reads; stats[5] = (long long)c->bg_used;
    }
    g53_lru_free(&t.c);
    return bad || t.overflow ? -1 : t.n;
}
