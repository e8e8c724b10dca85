/* g53h_lru.h - bookkeeping of the HBM expert cache: which expert key (layer * n_experts +
 * expert) sits in which slot, LRU order, pins, reads in flight and the prefetch queue.
 *
 * Pure C with no device calls, so the policy is testable on the CPU against the reference's
 * own cache (src/cache/glm53f_cache.c, compiled from its sources) on scripted traces. The
 * semantics restate the reference's:
 *   pick_victim   src/cache/glm53f_cache.c:55-66   (an EMPTY slot first, else the least
 *                                                   recently used one not pinned or in flight)
 *   reserve       src/cache/glm53f_cache.c:68-80
 *   land          src/cache/glm53f_cache.c:82-99
 *   get (hit)     src/cache/glm53f_cache.c:145-154
 *   release       src/cache/glm53f_cache.c:185-193
 *   hint          src/cache/glm53f_cache.c:251-293 (queue ordered by layer, stale entries of
 *                                                   layers below the floor and unlisted
 *                                                   entries of the hinted layer cancelled)
 *   pop           src/cache/glm53f_cache.c:299-306
 * The caller serialises every call (one mutex in the device cache). */
#ifndef G53H_LRU_H
#define G53H_LRU_H

#include <stdint.h>

#define G53_LRU_EMPTY    (-1)
#define G53_LRU_INFLIGHT (-2)

typedef struct {
    int       n_layers, n_experts, nslot;
    int32_t  *slot_of;        /* [n_layers * n_experts] -> resident slot or -1           */
    int32_t  *inflight_of;    /* [n_layers * n_experts] -> slot being filled or -1       */
    int32_t  *key_of;         /* [nslot] -> key, G53_LRU_EMPTY or G53_LRU_INFLIGHT        */
    int32_t  *pins;           /* [nslot] users; a pinned slot is never a victim           */
    unsigned char *prefetched;/* [nslot] filled by prefetch and not yet used              */
    uint64_t *used_at;        /* [nslot] LRU stamp                                       */
    uint64_t  clock;
    int32_t  *queue;          /* prefetch keys, ordered by layer                          */
    int       qcap, qlen, hint_floor, last_hint;
    unsigned char *queued;    /* [n_layers * n_experts]                                  */
    uint64_t  hits, misses, evictions, prefetch_reads, bg_reads, bg_used;
} G53hLru;

int  g53_lru_init(G53hLru *c, int n_layers, int n_experts, int nslot, int qcap);
void g53_lru_free(G53hLru *c);
int  g53_lru_pick_victim(const G53hLru *c);
/* Slot reserved for key (marked in flight), or -1 when every slot is pinned or in flight. */
int  g53_lru_reserve(G53hLru *c, int32_t key);
/* Publish (ok) or give back (failed) a reserved slot. */
void g53_lru_land(G53hLru *c, int32_t key, int slot, int ok, int background);
/* Hit path: the resident slot of key, pinned and stamped, or -1 when key is not resident. */
int  g53_lru_hit(G53hLru *c, int32_t key);
void g53_lru_release(G53hLru *c, int32_t key);
void g53_lru_hint(G53hLru *c, int layer, const int *ids, int n);
/* Next queued key that still needs a read (removed from the queue), or -1. */
int32_t g53_lru_pop(G53hLru *c);

#endif /* G53H_LRU_H */
