/* glm53f_st.h - the checkpoint index the expert cache reads experts through.
 *
 * The types are the reference's safetensors reader's (src/io/glm53f_st.h:24-58), field for
 * field, so a Glm53fSt opened by the reference's own glm53f_st_open can be handed to
 * glm53f_cache_init unchanged (tests/golden/offsets.json pins every offset). The cache only
 * reads the index (t[], nt) and the shard descriptors (fd[], dfd[]); it never calls the
 * reference reader's functions and builds its own name lookup over t[].
 *
 * For callers without the reference's reader (tests, benchmarks), g53h_st_open below is this
 * library's own reader of the same format: [8-byte little-endian N][N bytes of JSON header]
 * [tensor data], header entries {"dtype", "shape", "data_offsets": [start, end]} relative to
 * the end of the header. It fills a Glm53fSt the same way (absolute offsets, one descriptor per
 * shard, tensors in discovery order); bucket is left NULL, since nothing here uses it. */
#ifndef GLM53F_ST_H
#define GLM53F_ST_H

#include <stddef.h>
#include <stdint.h>

#include "glm53f.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum { GLM53F_DT_UNKNOWN = 0, GLM53F_DT_U8, GLM53F_DT_BF16, GLM53F_DT_F16, GLM53F_DT_F32,
               GLM53F_DT_F8_E4M3 } Glm53fDtype;

typedef struct {
    char       *name;
    int         shard;          /* index into Glm53fSt.fd[]                 */
    Glm53fDtype dtype;
    int         ndim;
    int64_t     shape[8];
    int64_t     off;            /* absolute byte offset within its shard    */
    int64_t     nbytes;
} Glm53fTensor;

/* Alignment of O_DIRECT reads (offset, length and buffer). */
#define GLM53F_ST_ALIGN 4096

typedef struct {
    int          *fd;           /* one open descriptor per shard            */
    int          *dfd;          /* the same shards opened O_DIRECT, or -1   */
    char        **path;
    int           nshard;
    Glm53fTensor *t;            /* every tensor, in discovery order         */
    int           nt;
    int32_t      *bucket;       /* the reference reader's name hash          */
    int           nbucket;
    char         *strpool;      /* names                                     */
    size_t        strcap, strlen_;
} Glm53fSt;

/* This library's reader (see above). Every *.safetensors file in dir, in name order, is one
 * shard. direct != 0 also opens each shard O_DIRECT (dfd), else dfd[] holds -1. Returns 0, or
 * -1 with a message on stderr. g53h_st_close closes and frees what g53h_st_open made. */
int  g53h_st_open(Glm53fSt *s, const char *dir, int direct);
void g53h_st_close(Glm53fSt *s);
/* Index of the tensor called name in s->t, or -1 (a linear scan: for tests and tools). */
int  g53h_st_index(const Glm53fSt *s, const char *name);

/* The bytes g53h_st_read_expert needs for one routed expert of cfg's shapes. */
size_t g53h_st_expert_bytes(const Glm53fCfg *cfg);
/* Read routed expert (layer, expert) from the checkpoint into host memory buf (cap bytes, at
 * least g53h_st_expert_bytes) the way the HBM cache stages it, and point q at it (FP8 views
 * into buf). 0, or -1 (missing or malformed tensors, short read, buf too small). */
int  g53h_st_read_expert(const Glm53fSt *st, const Glm53fCfg *cfg, int layer, int expert, void *buf, size_t cap,
                         Glm53fExpertQ *q);

#ifdef __cplusplus
}
#endif

#endif /* GLM53F_ST_H */
