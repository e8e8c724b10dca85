/* g53h_runtime.h - internal runtime state of the g53h library (one process, one device). */
#ifndef G53H_RUNTIME_H
#define G53H_RUNTIME_H

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "g53h.h"

extern "C" {
/* Record a failure message; returns -1 so callers can `return g53h_fail(...)`. */
int  g53h_fail(const char *fmt, ...);
/* Check a HIP status; on failure record it with the call site and return -1. */
int  g53h_check(hipError_t e, const char *what, const char *file, int line);
int  g53h_ready(void);         /* g53h_init(current) if needed; 0 ok            */
int  g53h_num_cus(void);
}
#define G53_TRY(call) do { if (g53h_check((call), #call, __FILE__, __LINE__)) return -1; } while (0)
/* Check the last kernel launch. */
#define G53_LAUNCHED(name) do { if (g53h_check(hipGetLastError(), name, __FILE__, __LINE__)) return -1; } while (0)

unsigned *g53h_mailbox_dev(void);    /* device address of the host mailbox             */
int g53h_current_device(void);        /* the device g53h_init bound, -1 before it      */
int g53_noalloc_setup(int device);    /* scratch address of the no-alloc decode (init)  */
hipStream_t g53h_stream(void);        /* compute stream; each call counts as an enqueue on it */
/* After enqueuing a kernel that writes sequence word `slot` of the mailbox last. */
void g53h_note_publish(int slot, unsigned seq);
/* 1 while the compute stream is quiet: a mailbox wait saw the last publication's sequence word
 * and nothing has been enqueued on the stream since. */
int g53h_quiet(void);
hipStream_t g53h_copy_stream(void);   /* side stream for host-to-HBM expert copies     */
/* g53h_tile_f8 on stream s (the expert cache tiles on its copy streams). */
int g53h_tile_f8_on(uint8_t *dst_d, const uint8_t *src_d, int rows, int cols, hipStream_t s);
int g53h_mtile_f8_on(uint8_t *dst_d, const uint8_t *src_d, int rows, int cols, int inverse, hipStream_t s);
int g53h_tile_i4_on(uint8_t *dst_d, const uint8_t *src_d, int rows, int cols, int inverse, hipStream_t s);
int g53h_mtile_i4_on(uint8_t *dw, float *ds, const uint8_t *sw, const float *ss, int rows, int cols, int inverse,
                     hipStream_t s);
int g53h_i4_from_f8_on(uint8_t *q_d, float *steps_d, const G53hMat *src, hipStream_t s);

/* Library workspace in HBM, grown on demand (grow = sync + free + alloc), 256-B aligned.
 * Regions are carved from it per call; nothing in it survives between calls except the
 * counters region, which kernels leave zeroed. */
void       *g53h_workspace(size_t bytes);
/* A zero-initialised region of 4096 ints that kernels use as arrival counters and flags and
 * always restore to zero before they exit. */
int        *g53h_counters(void);
/* The layer kernels' error flags, one int each ([0] k_dec_layer, [1] k_dec_tiled, [2] the
 * grouped path), zero at init; g53h_errors_async copies and clears them. */
int        *g53h_errblock(void);
/* The next layer's router scores of a decode token (g53h_route_next / g53h_decode_next): the
 * buffer [2][1024] (choice = score + bias, then score), and the request armed by
 * g53h_decode_next, which the tiled decode launch takes (its spare waves compute them) or
 * g53h_decode_publish serves with a launch of its own. */
struct G53NextReq {
    int armed;
    const float *x;
    const void *gate;
    int dt;
    const float *bias;
    int NE, E;
};
float      *g53h_next_buf(void);
G53NextReq *g53h_next_req(void);
/* Polls before a wait on another workgroup gives up (g53h_set_spin_limit). */
int         g53h_spin_limit(void);

/* Kernel timing marks (no-ops unless g53h_prof_enable(1)): tag 0 opens an interval, the
 * tags below close the interval since the previous mark. */
enum { G53_PROF_START = 0, G53_PROF_ROUTER = 1, G53_PROF_GATEUP = 2, G53_PROF_DOWN = 3,
       G53_PROF_GENERIC = 4, G53_PROF_GROUPED = 5, G53_PROF_COMBINE = 6, G53_PROF_FUSED = 7, G53_PROF_NTAGS = 8 };
void        g53h_prof_mark(int tag);

/* nw words from src to d by nt threads: 16 bytes a store where both are 16-byte aligned
 * (stores into host memory cross the link, and fewer, larger writes go faster), else 4. */
__device__ __forceinline__ void g53_copy_words(uint32_t *d, const uint32_t *src, int nw, int tid, int nt)
{
    if ((((uintptr_t)d | (uintptr_t)src) & 15) == 0) {
        const int n4 = nw >> 2;
        for (int i = tid; i < n4; i += nt) ((uint4 *)d)[i] = ((const uint4 *)src)[i];
        for (int i = 4 * n4 + tid; i < nw; i += nt) d[i] = src[i];
    } else {
        for (int i = tid; i < nw; i += nt) d[i] = src[i];
    }
}

#endif /* G53H_RUNTIME_H */
