/* glm53f_i4file.h - the int4 expert container on disk (the reference's --write-int4 and
 * --int4-dir), implemented by glm-5.3-flash-in-c_amd/host/g53h_i4file.c.
 *
 * Replaces: include/glm53f/glm53f_i4file.h with src/io/glm53f_i4file.c (same declarations,
 * same file format, byte for byte). One file per MoE layer, <dir>/layer-LL.i4:
 *   [4096-byte header][expert 0][expert 1]...[expert n-1]
 * every expert exactly an int4 cache slot (src/io/glm53f_load.c:141-163), so a read lands in
 * the slot as it is. The header carries a fingerprint of the checkpoint the layer was written
 * from, a CRC-32 per expert and a completion mark written last. glm53f_cache_init with i4 != 0
 * reads the layers found in glm53f_i4_dir (include/glm53f.h) instead of quantising them. */
#ifndef GLM53F_I4FILE_H
#define GLM53F_I4FILE_H

#include <stdint.h>

#include "glm53f.h"
#include "glm53f_st.h"

#ifdef __cplusplus
extern "C" {
#endif

#define GLM53F_I4F_HEADER 4096

/* Write one MoE layer's experts to <dir>/layer-LL.i4 (the experts quantised on the device).
 * Skips a layer already complete and valid. Returns 0 on success, 1 when skipped, -1 on failure
 * (the .part file is removed). Reference: glm53f_i4file.h:33-35. */
int glm53f_i4file_write_layer(const Glm53fSt *st, const Glm53fCfg *c, int layer, const char *dir);

/* Open <dir>/layer-LL.i4 for reading experts: a descriptor, -1 when there is no file, -2 when a
 * file is there but does not belong to this checkpoint or is incomplete (a message says why).
 * Reference: glm53f_i4file.h:37-40. */
int glm53f_i4file_open_layer(const Glm53fSt *st, const Glm53fCfg *c, int layer, const char *dir);

/* Verify every expert of a layer against its CRC: the number of bad experts, or -1 when the
 * file cannot be read. Reference: glm53f_i4file.h:42-44. */
int glm53f_i4file_verify_layer(const Glm53fSt *st, const Glm53fCfg *c, int layer, const char *dir);

/* Offset of an expert inside its layer file. Reference: glm53f_i4file.h:46-50. */
static inline int64_t glm53f_i4file_offset(int expert, int64_t slot_bytes)
{
    return GLM53F_I4F_HEADER + (int64_t)expert * slot_bytes;
}

#ifdef __cplusplus
}
#endif
#endif /* GLM53F_I4FILE_H */
