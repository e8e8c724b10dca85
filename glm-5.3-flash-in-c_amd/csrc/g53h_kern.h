/* g53h_kern.h - declarations shared between the library's HIP translation units. */
#ifndef G53H_KERN_H
#define G53H_KERN_H

#include "g53h.h"

#define GLM53F_MAX_TOPK_DEV 64

/* The experts of a layer by the row-wave kernels (int4, and FP8 of any geometry): act [T][nslots][I]
 * = swiglu(gate . x, up . x), contrib [T][nslots][E] = down . act, for descriptors slots [T][nslots]. */
int g53h_rows_layer(float *contrib, float *act, const float *x, int T, int nslots, const G53hExpert *slots, int E,
                    int I, float limit);
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
int g53h_decode_mtiled(float *out, const float *x, const G53hMoeLayer *L, int *idx_out, float *w_out,
                       const int *idx_in, const float *w_in);
int g53h_grouped_use(const G53hMoeLayer *L, int T);
int g53h_swiglu_split(float *y, const float *g, const float *u, long m, float limit);

#endif /* G53H_KERN_H */
