/* Test infrastructure: the reference's own expert cache (src/cache/glm53f_cache.c, compiled
 * from its source file in this translation unit, so its static policy functions are callable)
 * driven by a scripted trace over a checkpoint directory (the reference's glm_tiny fixture).
 * The trace format and outputs are those of g53h_lru_trace in the library:
 *   1 L E get, 2 L E release, 3 L n e... getmany, 4 L n e... hint, 5 k serve k background reads.
 * The cache is created with no I/O threads; hint() is enabled by setting n_io afterwards, and
 * "serve" runs the body of the reference's io_main (src/cache/glm53f_cache.c:297-319) inline,
 * so the trace is deterministic. */
#include "glm53f_cache.c"
#include "glm53f_cfg.h"

#include <stdio.h>

int ref_cache_trace(const char *model_dir, int nslot, const int *ops, int nops, int *out, int outcap,
                    long long *stats, int *n_layers_out, int *n_experts_out)
{
    static Glm53fSt st;
    static Glm53fCfg cfg;
    char path[4096];
    snprintf(path, sizeof path, "%s/config.json", model_dir);
    if (!glm53f_cfg_load_file(&cfg, path)) return -1;
    if (glm53f_st_open(&st, model_dir) != 0) return -1;
    int probe = -1;
    for (int L = 0; L < cfg.n_layers; L++) if (!glm53f_is_dense(&cfg, L)) { probe = L; break; }
    Glm53fExpertRef r;
    if (probe < 0 || glm53f_expert_ref(&st, &cfg, probe, 0, &r) != 0) { glm53f_st_close(&st); return -1; }
    const int64_t slot_bytes = glm53f_expert_slot_bytes(&r) + GLM53F_ST_ALIGN;
    Glm53fCache c;
    if (glm53f_cache_init(&c, &st, &cfg, (int64_t)nslot * slot_bytes, 0, 0) != 0) { glm53f_st_close(&st); return -1; }
    c.n_io = 1;                                  /* hint() edits the queue; no thread reads it */
    *n_layers_out = c.n_layers;
    *n_experts_out = c.n_experts;
    int o = 0, bad = 0;
#define PUT(v) do { if (o >= outcap) { bad = 1; goto end; } out[o++] = (v); } while (0)
    for (int i = 0; i < nops;) {
        const int op = ops[i++];
        if (op == 1) {
            const int L = ops[i++], e = ops[i++];
            int was = 0;
            if (L >= 0 && L < c.n_layers && e >= 0 && e < c.n_experts) was = c.slot_of[L * c.n_experts + e] >= 0;
            Glm53fExpertQ q;
            const int rc = c.src.get(&c.src, L, e, &q);
            PUT(rc);
            PUT(was);
            PUT(rc == 0 ? (int)(((const unsigned char *)q.gate.w - c.arena) / c.slot_bytes) : -1);
        } else if (op == 2) {
            const int L = ops[i++], e = ops[i++];
            c.src.release(&c.src, L, e);
        } else if (op == 3) {
            const int L = ops[i++], n = ops[i++];
            PUT(c.src.getmany(&c.src, L, ops + i, n));
            i += n;
        } else if (op == 4) {
            const int L = ops[i++], n = ops[i++];
            c.src.hint(&c.src, L, ops + i, n);
            i += n;
            PUT(c.qlen);
            for (int k = 0; k < c.qlen; k++) PUT(c.queue[k]);
        } else if (op == 5) {
            const int k = ops[i++];
            for (int rd = 0; rd < k;) {
                if (c.qlen == 0) break;
                const int32_t key = c.queue[0];
                memmove(c.queue, c.queue + 1, (size_t)(c.qlen - 1) * sizeof *c.queue);
                c.qlen--;
                c.queued[key] = 0;
                if (c.slot_of[key] >= 0 || c.inflight_of[key] >= 0) continue;
                const int slot = reserve(&c, key);
                if (slot < 0) continue;
                Glm53fExpertRef rr;
                int64_t pad, nread;
                const int ok = load_into(&c, key / c.n_experts, key % c.n_experts, slot, &rr, &pad, &nread);
                land(&c, key, slot, &rr, pad, ok, 1);
                if (ok) { c.bg_reads++; c.bg_bytes += (uint64_t)nread; }
                PUT(key);
                PUT(slot);
                rd++;
            }
            PUT(-1);
        } else {
            bad = 1;
            break;
        }
    }
end:
#undef PUT
    stats[0] = (long long)c.hits; stats[1] = (long long)c.misses; stats[2] = (long long)c.evictions;
    stats[3] = (long long)c.prefetch_reads; stats[4] = (long long)c.bg_reads; stats[5] = (long long)c.bg_used;
    c.n_io = 0;
    glm53f_cache_free(&c);
    glm53f_st_close(&st);
    return bad ? -1 : o;
}
