/* g53h_ckpt.h - routed experts read from a checkpoint index (Glm53fSt) into pinned staging
 * buffers, for the HBM expert cache (g53h_ckpt.c). */
#ifndef G53H_CKPT_H
#define G53H_CKPT_H

#include "glm53f.h"
#include "glm53f_st.h"

#ifdef __cplusplus
extern "C" {
#endif

#define G53H_CKPT_BUSY (-2)        /* every staging buffer holds an expert not yet done */

typedef struct G53hCkpt G53hCkpt;

/* The expert table of st for layers [0, n_layers) and nstage pinned staging buffers. NULL on
 * failure. */
G53hCkpt *g53h_ckpt_new(const Glm53fSt *st, const Glm53fCfg *cfg, int n_layers, int nstage);
void      g53h_ckpt_free(G53hCkpt *k);
/* Read expert (layer, expert) into a free staging buffer and point q at it (FP8 views).
 * 0, -1 (missing, malformed or short read), or G53H_CKPT_BUSY. */
int       g53h_ckpt_view(G53hCkpt *k, int layer, int expert, Glm53fExpertQ *q);
/* The buffer holding (layer, expert) is free again. */
void      g53h_ckpt_done(G53hCkpt *k, int layer, int expert);

#ifdef __cplusplus
}
#endif

#endif /* G53H_CKPT_H */
