/* g53h_kern.h - declarations shared between the library's HIP translation units. */
#ifndef G53H_KERN_H
#define G53H_KERN_H

#include "g53h.h"

#define GLM53F_MAX_TOPK_DEV 64

/* y [T][nslots][rows] = matrix `which` (0 gate, 1 up, 2 down) of slots[t][s] times x (per
 * token, or per (token, slot) when x_per_slot) by the row-wave kernel (any FP8 geometry, int4). */
int g53h_slot_rows(float *y, const float *x, int T, int nslots, const G53hExpert *slots, int which, int rows,
                   int cols, int x_per_slot);
int g53h_combine_into(float *out, const float *contrib, const float *wts, int T, int E, int K, int nslots);
int g53h_resolve_slots(G53hExpert *slots, const G53hExpert *experts, const int *idx, const G53hExpert *shared,
                       int T, int K);
int g53h_router_into(int *idx, float *w, const float *x, int T, const void *gate, int gate_dt,
                     const float *bias, int NE, int E, int K, int norm_topk, float routed_scale,
                     int *nan_flag, float *scratch, const G53hExpert *experts, const G53hExpert *shared,
                     G53hExpert *slots);
int g53h_decode_fused(float *out, const float *x, const G53hMoeLayer *L, int *idx_out, float *w_out);
int g53h_decode_tiled(float *out, const float *x, const G53hMoeLayer *L, int *idx_out, float *w_out,
                      const int *idx_in, const float *w_in);
int g53h_decode_tiled_grid(void);
int g53h_grouped_use(const G53hMoeLayer *L, int T);
int g53h_swiglu_split(float *y, const float *g, const float *u, long m, float limit);

#endif /* G53H_KERN_H */
