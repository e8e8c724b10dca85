/* g53h_lru.c - see g53h_lru.h. */
#include "g53h_lru.h"

#include <stdlib.h>
#include <string.h>

int g53_lru_init(G53hLru *c, int n_layers, int n_experts, int nslot, int qcap)
{
    memset(c, 0, sizeof *c);
    if (n_layers < 1 || n_experts < 1 || nslot < 1 || qcap < 1) return -1;
    const size_t nkey = (size_t)n_layers * (size_t)n_experts;
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
    c->queue = (int32_t *)malloc((size_t)qcap * sizeof(int32_t));
    if (!c->slot_of || !c->inflight_of || !c->queued || !c->key_of || !c->pins || !c->prefetched ||
        !c->used_at || !c->queue) {
        g53_lru_free(c);
        return -1;
    }
    for (size_t i = 0; i < nkey; i++) { c->slot_of[i] = -1; c->inflight_of[i] = -1; }
    for (int i = 0; i < nslot; i++) c->key_of[i] = G53_LRU_EMPTY;
    c->last_hint = -1;
    return 0;
}

void g53_lru_free(G53hLru *c)
{
    free(c->slot_of); free(c->inflight_of); free(c->queued); free(c->key_of); free(c->pins);
    free(c->prefetched); free(c->used_at); free(c->queue);
    memset(c, 0, sizeof *c);
}

int g53_lru_pick_victim(const G53hLru *c)
{
    int best = -1;
    uint64_t oldest = UINT64_MAX;
    for (int i = 0; i < c->nslot; i++) {
        if (c->key_of[i] == G53_LRU_INFLIGHT || c->pins[i] > 0) continue;
        if (c->key_of[i] == G53_LRU_EMPTY) return i;
        if (c->used_at[i] < oldest) { oldest = c->used_at[i]; best = i; }
    }
    return best;
}

int g53_lru_reserve(G53hLru *c, int32_t key)
{
    const int slot = g53_lru_pick_victim(c);
    if (slot < 0) return -1;
    if (c->key_of[slot] >= 0) { c->slot_of[c->key_of[slot]] = -1; c->evictions++; }
    c->key_of[slot] = G53_LRU_INFLIGHT;
    c->prefetched[slot] = 0;
    c->inflight_of[key] = slot;
    return slot;
}

void g53_lru_land(G53hLru *c, int32_t key, int slot, int ok, int background)
{
    c->inflight_of[key] = -1;
    if (ok) {
        c->key_of[slot] = key;
        c->slot_of[key] = slot;
        c->used_at[slot] = ++c->clock;
        c->prefetched[slot] = (unsigned char)(background != 0);
    } else {
        c->key_of[slot] = G53_LRU_EMPTY;
    }
}

int g53_lru_hit(G53hLru *c, int32_t key)
{
    const int slot = c->slot_of[key];
    if (slot < 0) return -1;
    c->hits++;
    if (c->prefetched[slot]) { c->bg_used++; c->prefetched[slot] = 0; }
    c->used_at[slot] = ++c->clock;
    c->pins[slot]++;
    return slot;
}

void g53_lru_release(G53hLru *c, int32_t key)
{
    const int slot = c->slot_of[key];
    if (slot >= 0 && c->pins[slot] > 0) c->pins[slot]--;
}

void g53_lru_hint(G53hLru *c, int layer, const int *ids, int n)
{
    if (layer < 0 || layer >= c->n_layers) return;
    if (layer <= c->last_hint) c->hint_floor = layer;
    c->last_hint = layer;
    int kept = 0;
    for (int i = 0; i < c->qlen; i++) {
        const int32_t key = c->queue[i];
        const int kl = key / c->n_experts;
        int drop = kl < c->hint_floor;
        if (kl == layer) {
            drop = 1;
            for (int j = 0; j < n; j++)
                if (ids[j] == key % c->n_experts) { drop = 0; break; }
        }
        if (drop) { c->queued[key] = 0; continue; }
        c->queue[kept++] = key;
    }
    c->qlen = kept;
    int at = c->qlen;                      /* after every pending entry of a layer <= `layer` */
    while (at > 0 && c->queue[at - 1] / c->n_experts > layer) at--;
    for (int i = 0; i < n && c->qlen < c->qcap; i++) {
        const int e = ids[i];
        if (e < 0 || e >= c->n_experts) continue;
        const int32_t key = layer * c->n_experts + e;
        if (c->queued[key] || c->slot_of[key] >= 0 || c->inflight_of[key] >= 0) continue;
        c->queued[key] = 1;
        memmove(c->queue + at + 1, c->queue + at, (size_t)(c->qlen - at) * sizeof *c->queue);
        c->queue[at++] = key;
        c->qlen++;
    }
}

int32_t g53_lru_pop(G53hLru *c)
{
    while (c->qlen > 0) {
        const int32_t key = c->queue[0];
        memmove(c->queue, c->queue + 1, (size_t)(c->qlen - 1) * sizeof *c->queue);
        c->qlen--;
        c->queued[key] = 0;
        if (c->slot_of[key] >= 0 || c->inflight_of[key] >= 0) continue;
        return key;
    }
    return -1;
}

/* ----------------------------------------------------------- scripted traces ---- */
#include "glm53f_cache.h"

#define G53_LRU_QCAP (64 * 4 * GLM53F_MAX_TOPK)   /* the reference's queue capacity */

int g53h_lru_trace(int n_layers, int n_experts, int nslot, const int *ops, int nops, int *out, int outcap,
                   long long *stats)
{
    G53hLru c;
    if (g53_lru_init(&c, n_layers, n_experts, nslot, G53_LRU_QCAP)) return -1;
    int o = 0, bad = 0;
#define PUT(v) do { if (o >= outcap) { bad = 1; goto end; } out[o++] = (v); } while (0)
    for (int i = 0; i < nops;) {
        const int op = ops[i++];
        if (op == 1 || op == 2) {                       /* get / release */
            const int L = ops[i++], e = ops[i++];
            if (L < 0 || L >= n_layers || e < 0 || e >= n_experts) {
                if (op == 1) { PUT(-1); PUT(0); PUT(-1); }
                continue;
            }
            const int32_t key = L * n_experts + e;
            if (op == 2) { g53_lru_release(&c, key); continue; }
            const int was = c.slot_of[key] >= 0;
            int slot = g53_lru_hit(&c, key);
            if (slot < 0) {
                c.misses++;
                const int s = g53_lru_reserve(&c, key);
                if (s < 0) { c.misses--; PUT(-1); PUT(was); PUT(-1); continue; }
                g53_lru_land(&c, key, s, 1, 0);
                slot = g53_lru_hit(&c, key);
                c.hits--;                               /* the read, not a hit */
            }
            PUT(0); PUT(was); PUT(slot);
        } else if (op == 3) {                           /* getmany */
            const int L = ops[i++], n = ops[i++];
            const int *ids = ops + i;
            i += n;
            int keys[GLM53F_MAX_TOPK], slots[GLM53F_MAX_TOPK], nw = 0;
            for (int j = 0; j < n && nw < GLM53F_MAX_TOPK; j++) {
                const int e = ids[j];
                if (e < 0 || e >= n_experts || L < 0 || L >= n_layers) continue;
                const int32_t key = L * n_experts + e;
                if (c.slot_of[key] >= 0 || c.inflight_of[key] >= 0) continue;
                const int s = g53_lru_reserve(&c, key);
                if (s < 0) break;
                keys[nw] = key; slots[nw] = s; nw++;
            }
            for (int k = 0; k < nw; k++) { g53_lru_land(&c, keys[k], slots[k], 1, 0); c.prefetch_reads++; }
            PUT(nw);
        } else if (op == 4) {                           /* hint */
            const int L = ops[i++], n = ops[i++];
            g53_lru_hint(&c, L, ops + i, n);
            i += n;
            PUT(c.qlen);
            for (int k = 0; k < c.qlen; k++) PUT(c.queue[k]);
        } else if (op == 5) {                           /* serve up to k background reads */
            const int k = ops[i++];
            for (int r = 0; r < k;) {
                const int32_t key = g53_lru_pop(&c);
                if (key < 0) break;
                const int s = g53_lru_reserve(&c, key);
                if (s < 0) continue;                    /* cache saturated: the hint is skipped */
                g53_lru_land(&c, key, s, 1, 1);
                c.bg_reads++;
                PUT(key); PUT(s);
                r++;
            }
            PUT(-1);
        } else {
            bad = 1;
            break;
        }
    }
end:
#undef PUT
    if (stats) {
        stats[0] = (long long)c.hits; stats[1] = (long long)c.misses; stats[2] = (long long)c.evictions;
        stats[3] = (long long)c.prefetch_reads; stats[4] = (long long)c.bg_reads; stats[5] = (long long)c.bg_used;
    }
    g53_lru_free(&c);
    return bad ? -1 : o;
}
