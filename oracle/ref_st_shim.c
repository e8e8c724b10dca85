/* Test infrastructure: the reference's safetensors reader and expert loader
 * (src/io/glm53f_st.c, src/io/glm53f_load.c, compiled from their sources into
 * _ref/libglm53f_ref.so) on a checkpoint directory, to pin this library's reader
 * (g53h_st_open) and expert staging (g53h_st_read_expert) on the same files. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "glm53f.h"
#include "glm53f_load.h"
#include "glm53f_st.h"

/* The reference's index of dir: per tensor (discovery order) 7 int64 (shard, dtype, ndim,
 * shape[0], shape[1], off, nbytes) into meta, names '\n'-separated into names. Returns the
 * tensor count, or -1. */
int ref_st_table(const char *dir, long long *meta, int cap, char *names, int names_cap)
{
    Glm53fSt st;
    if (glm53f_st_open(&st, dir) != 0) return -1;
    int n = st.nt < cap ? st.nt : cap, o = 0;
    for (int i = 0; i < n; i++) {
        const Glm53fTensor *t = &st.t[i];
        long long *m = meta + 7 * i;
        m[0] = t->shard; m[1] = t->dtype; m[2] = t->ndim;
        m[3] = t->ndim > 0 ? t->shape[0] : 0; m[4] = t->ndim > 1 ? t->shape[1] : 0;
        m[5] = t->off; m[6] = t->nbytes;
        const int l = (int)strlen(t->name);
        if (o + l + 1 < names_cap) { memcpy(names + o, t->name, (size_t)l); o += l; names[o++] = '\n'; }
    }
    names[o < names_cap ? o : names_cap - 1] = 0;
    glm53f_st_close(&st);
    return n;
}

/* Routed expert (layer, expert) read by the reference's loader (glm53f_expert_ref, _load and
 * _view), copied out as gate, up, down codes then gate, up, down scales. Returns the bytes
 * written, or -1. */
long long ref_expert_read(const char *dir, int hidden, int inter, int n_experts, int br, int bc, int layer,
                          int expert, uint8_t *out, long long cap)
{
    Glm53fSt st;
    if (glm53f_st_open(&st, dir) != 0) return -1;
    Glm53fCfg c;
    memset(&c, 0, sizeof c);
    c.hidden = hidden; c.moe_inter = inter; c.n_experts = n_experts; c.fp8_block_r = br; c.fp8_block_c = bc;
    Glm53fExpertRef r;
    long long o = -1;
    if (glm53f_expert_ref(&st, &c, layer, expert, &r) == 0) {
        const int64_t sb = glm53f_expert_slot_bytes(&r);
        unsigned char *slot = NULL;
        if (posix_memalign((void **)&slot, GLM53F_ST_ALIGN, (size_t)sb + GLM53F_ST_ALIGN) == 0) {
            int64_t pad = 0;
            if (glm53f_expert_load(&st, &r, slot, sb + GLM53F_ST_ALIGN, &pad) == 0) {
                Glm53fExpertQ q;
                glm53f_expert_view(&r, &c, slot, pad, glm53f_expert_weight_area(&r), &q);
                const Glm53fMat *m[3] = {&q.gate, &q.up, &q.down};
                o = 0;
                for (int i = 0; i < 3 && o >= 0; i++) {
                    const long long n = (long long)m[i]->rows * m[i]->cols;
                    if (o + n > cap) { o = -1; break; }
                    memcpy(out + o, m[i]->w, (size_t)n);
                    o += n;
                }
                for (int i = 0; i < 3 && o >= 0; i++) {
                    const long long n = (long long)((m[i]->rows + br - 1) / br) * m[i]->scols * 4;
                    if (o + n > cap) { o = -1; break; }
                    memcpy(out + o, m[i]->s, (size_t)n);
                    o += n;
                }
            }
            free(slot);
        }
    }
    glm53f_st_close(&st);
    return o;
}
