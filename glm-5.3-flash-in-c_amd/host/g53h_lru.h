/* g53h_lru.h - bookkeeping of the HBM expert cache: which expert key (layer * n_experts +
 * expert) sits in which slot, the eviction order, pins, reads in flight and the prefetch queue.
 *
 * Pure C with no device calls, so the policy is testable on the CPU against the reference's
 * own cache (src/cache/glm53f_cache.c, compiled from its sources) on scripted traces. The
 * decisions are the reference's (src/cache/glm53f_cache.c:55-99 victim choice, reservation and
 * landing; :145-154 hit; :185-193 release; :251-293 hint; :299-306 the reader's dequeue); the
 * data structures are this file's own, sized for an HBM cache of thousands of slots:
 *
 *   victim choice   an EMPTY slot first, lowest index: a two-level bitmap, found in two
 *                   count-trailing-zero steps; otherwise the least recently used slot that is
 *                   neither pinned nor being filled: an indexed binary min-heap keyed by the
 *                   slot's use stamp, holding exactly the resident, unpinned slots. A slot
 *                   leaves the heap when it is pinned or chosen and re-enters when its last pin
 *                   is released or its read lands, so every operation is O(log nslot) instead
 *                   of a scan over all slots.
 *   prefetch queue  one FIFO per layer (singly linked nodes from a fixed pool), read lowest
 *                   layer first: appending a hint is O(1), cancelling a layer below the floor
 *                   drops its whole list, and filtering the hinted layer's list by the new ids
 *                   uses a per-expert mark instead of a search of the id list.
 *
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
    uint64_t *used_at;        /* [nslot] use stamp                                       */
    uint64_t  clock;
    /* victims */
    uint64_t *empty_w;        /* bit s: slot s is EMPTY                                   */
    uint64_t *empty_s;        /* bit w: word w of empty_w is non-zero                     */
    int32_t  *heap;           /* evictable slots, heap-ordered by used_at                 */
    int32_t  *heap_at;        /* [nslot] position in heap, or -1                          */
    int       heap_n;
    /* prefetch queue */
    int32_t  *q_key, *q_next; /* node pool [qcap]                                          */
    int32_t  *q_head, *q_tail;/* [n_layers] per-layer lists, -1 when empty                 */
    int32_t   q_free;         /* free-node list                                            */
    int       q_lo;           /* no layer below q_lo has queued entries                    */
    int32_t  *mark;           /* [n_experts] hint stamp of the ids being hinted            */
    int32_t   mark_gen;
    int       qcap, qlen, hint_floor, last_hint;
    unsigned char *queued;    /* [n_layers * n_experts]                                  */
    uint64_t  hits, misses, evictions, prefetch_reads, bg_reads, bg_used;
} G53hLru;

int  g53_lru_init(G53hLru *c, int n_layers, int n_experts, int nslot, int qcap);
void g53_lru_free(G53hLru *c);
/* The slot the next reservation would take, or -1 when every slot is pinned or in flight. */
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
/* The queued keys in the order they would be read; returns how many were written (<= cap). */
int  g53_lru_queue(const G53hLru *c, int32_t *keys, int cap);

#endif /* G53H_LRU_H */
