/* g53h_i4file.c - the int4 expert container on disk (include/glm53f_i4file.h), the format of
 * the reference's src/io/glm53f_i4file.c (--write-int4, --int4-dir):
 *
 *   <dir>/layer-LL.i4 = [4096-byte header][expert 0][expert 1]...[expert n-1]
 *   header: bytes 0-7 "GLM53FI4", u32 version 1 at 8, u32 layer at 12, u32 n_experts at 16,
 *           u32 group (64) at 20, u64 slot_bytes at 24, u64 checkpoint fingerprint at 32,
 *           u32 completion mark (1) at 40, u32 CRC-32 of expert e at 48 + 4 e;
 *   expert: slot_bytes, exactly an int4 cache slot (src/io/glm53f_load.c:141-163: per matrix
 *           the packed levels, then the fp32 steps, each 64-byte aligned; rounded to 4096).
 *
 * The fingerprint (src/io/glm53f_i4file.c:47-72) ties a file to the checkpoint it came from:
 * FNV-1a (64-bit, each value's 8 little-endian bytes) over the layer, the geometry, the group,
 * and for experts 0 and n-1 where their tensors sit (shard, weights run offset and size,
 * scales run offset, matrix shapes) and the slot size. The writer quantises on the device
 * (g53h_i4_from_f8, bit-exact with the reference's glm53f_i4_from_f8), so a file it writes is
 * byte-identical to the reference's. A file from another checkpoint, of another version or
 * without its completion mark is refused; a writer that stops midway leaves only a .part file. */
#define _GNU_SOURCE
#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "g53h.h"
#include "glm53f.h"
#include "glm53f_i4file.h"
#include "glm53f_st.h"

const char *glm53f_i4_dir = NULL;

#define I4F_VERSION 1
static const char I4F_MAGIC[8] = {'G', 'L', 'M', '5', '3', 'F', 'I', '4'};

/* CRC-32 of IEEE 802.3 (reflected polynomial 0xEDB88320, initial and final xor ~0). */
static uint32_t g_crc_tab[256];
static uint32_t crc32_of(const uint8_t *p, size_t n)
{
    if (!g_crc_tab[1])
        for (uint32_t i = 0; i < 256; i++) {
            uint32_t v = i;
            for (int k = 0; k < 8; k++) v = (v >> 1) ^ (0xEDB88320u & (0u - (v & 1u)));
            g_crc_tab[i] = v;
        }
    uint32_t v = ~0u;
    for (size_t i = 0; i < n; i++) v = g_crc_tab[(v ^ p[i]) & 0xffu] ^ (v >> 8);
    return ~v;
}

/* FNV-1a, 64-bit, over the 8 little-endian bytes of v. */
static uint64_t fnv_i64(uint64_t h, int64_t v)
{
    const uint64_t u = (uint64_t)v;
    for (int i = 0; i < 8; i++) {
        h ^= (u >> (8 * i)) & 0xffu;
        h *= 1099511628211ull;
    }
    return h;
}

static void le32(uint8_t *p, uint32_t v) { for (int i = 0; i < 4; i++) p[i] = (uint8_t)(v >> (8 * i)); }
static void le64(uint8_t *p, uint64_t v) { for (int i = 0; i < 8; i++) p[i] = (uint8_t)(v >> (8 * i)); }
static uint32_t rd32(const uint8_t *p) { uint32_t v = 0; for (int i = 3; i >= 0; i--) v = v << 8 | p[i]; return v; }
static uint64_t rd64(const uint8_t *p) { uint64_t v = 0; for (int i = 7; i >= 0; i--) v = v << 8 | p[i]; return v; }

/* Matrix m of an expert (0 gate, 1 up, 2 down): rows x cols. */
static void mat_shape(const Glm53fCfg *c, int m, int *rows, int *cols)
{
    *rows = m < 2 ? c->moe_inter : c->hidden;
    *cols = m < 2 ? c->hidden : c->moe_inter;
}

/* Byte offsets of matrix m's levels and steps in an int4 slot; returns the slot's size. */
static int64_t i4_slot(const Glm53fCfg *c, int64_t qoff[3], int64_t soff[3])
{
    int64_t o = 0;
    for (int m = 0; m < 3; m++) {
        int rows, cols;
        mat_shape(c, m, &rows, &cols);
        o = (o + 63) & ~(int64_t)63;
        qoff[m] = o;
        o += (int64_t)rows * (cols / 2);
        o = (o + 63) & ~(int64_t)63;
        soff[m] = o;
        o += (int64_t)rows * (cols / GLM53F_I4_GROUP) * 4;
    }
    return (o + GLM53F_ST_ALIGN - 1) / GLM53F_ST_ALIGN * GLM53F_ST_ALIGN;
}

/* An expert's six tensors (weights, then scale grids) by the checkpoint's names, the reference's
 * "model.language_model.layers.L.mlp.experts.E.P_proj.weight[_scale_inv]". */
static int expert_tensors(const Glm53fSt *st, int layer, int expert, const Glm53fTensor *t[6])
{
    static const char *P[3] = {"gate", "up", "down"};
    char name[256];
    for (int k = 0; k < 6; k++) {
        snprintf(name, sizeof name, "model.language_model.layers.%d.mlp.experts.%d.%s_proj.%s", layer, expert,
                 P[k % 3], k < 3 ? "weight" : "weight_scale_inv");
        const int i = g53h_st_index(st, name);
        if (i < 0) return -1;
        t[k] = &st->t[i];
    }
    return 0;
}

/* What the fingerprint hashes of one expert (src/io/glm53f_load.c:64-95): when the three
 * weights are one run and the three scale grids another, all in one shard, that shard and the
 * runs' offsets; otherwise zeros. w_bytes is the weights' total either way. */
static int expert_fp(const Glm53fSt *st, const Glm53fCfg *c, int layer, int expert, uint64_t h, uint64_t *out)
{
    const Glm53fTensor *t[6];
    if (expert_tensors(st, layer, expert, t)) return -1;
    const int shard = t[0]->shard;
    int same = 1;
    int64_t wlo = t[0]->off, whi = 0, wown = 0, slo = -1, shi = 0, sown = 0;
    for (int m = 0; m < 3; m++) {
        int rows, cols;
        mat_shape(c, m, &rows, &cols);
        if (t[m]->ndim != 2 || t[m]->shape[0] != rows || t[m]->shape[1] != cols || t[m]->dtype != GLM53F_DT_F8_E4M3)
            return -1;
        if (t[m]->shard != shard || t[3 + m]->shard != shard) same = 0;
        if (t[m]->off < wlo) wlo = t[m]->off;
        if (t[m]->off + t[m]->nbytes > whi) whi = t[m]->off + t[m]->nbytes;
        wown += t[m]->nbytes;
        if (slo < 0 || t[3 + m]->off < slo) slo = t[3 + m]->off;
        if (t[3 + m]->off + t[3 + m]->nbytes > shi) shi = t[3 + m]->off + t[3 + m]->nbytes;
        sown += t[3 + m]->nbytes;
    }
    const int contiguous = same && whi - wlo == wown && shi - slo == sown;
    h = fnv_i64(h, contiguous ? shard : 0);
    h = fnv_i64(h, contiguous ? wlo : 0);
    h = fnv_i64(h, wown);
    h = fnv_i64(h, contiguous ? slo : 0);
    for (int m = 0; m < 3; m++) {
        int rows, cols;
        mat_shape(c, m, &rows, &cols);
        h = fnv_i64(h, rows);
        h = fnv_i64(h, cols);
    }
    *out = h;
    return 0;
}

static int fingerprint(const Glm53fSt *st, const Glm53fCfg *c, int layer, int64_t *slot_bytes, uint64_t *fp)
{
    int64_t qo[3], so[3];
    *slot_bytes = i4_slot(c, qo, so);
    uint64_t h = 1469598103934665603ull;
    h = fnv_i64(h, layer); h = fnv_i64(h, c->n_experts); h = fnv_i64(h, c->hidden); h = fnv_i64(h, c->moe_inter);
    h = fnv_i64(h, c->fp8_block_r); h = fnv_i64(h, c->fp8_block_c); h = fnv_i64(h, GLM53F_I4_GROUP);
    const int probe[2] = {0, c->n_experts - 1};
    for (int i = 0; i < 2; i++)
        if (expert_fp(st, c, layer, probe[i], h, &h)) return -1;
    *fp = fnv_i64(h, *slot_bytes);
    return 0;
}

static void layer_path(char *buf, size_t cap, const char *dir, int layer, const char *suffix)
{
    snprintf(buf, cap, "%s/layer-%02d.i4%s", dir, layer, suffix);
}

/* The layer's file checked against this checkpoint: its descriptor, -1 when absent, -2 when
 * unusable (why on stderr unless quiet). hdr (GLM53F_I4F_HEADER bytes) receives the header. */
static int open_checked(const Glm53fSt *st, const Glm53fCfg *c, int layer, const char *dir, int64_t *slot,
                        uint8_t *hdr, int quiet)
{
    char path[1024];
    layer_path(path, sizeof path, dir, layer, "");
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return -1;
    uint64_t fp = 0;
    const char *why = NULL;
    if (pread(fd, hdr, GLM53F_I4F_HEADER, 0) != GLM53F_I4F_HEADER) why = "short header";
    else if (memcmp(hdr, I4F_MAGIC, 8)) why = "not an int4 container";
    else if (rd32(hdr + 8) != I4F_VERSION) why = "another container version";
    else if (rd32(hdr + 40) != 1) why = "incomplete";
    else if ((int)rd32(hdr + 12) != layer || (int)rd32(hdr + 16) != c->n_experts || rd32(hdr + 20) != GLM53F_I4_GROUP)
        why = "another layer or geometry";
    else if (fingerprint(st, c, layer, slot, &fp)) why = "the checkpoint layer cannot be resolved";
    else if ((int64_t)rd64(hdr + 24) != *slot || rd64(hdr + 32) != fp) why = "written from another checkpoint";
    if (why) {
        if (!quiet)
            fprintf(stderr, "glm53f: %s is not usable (%s); layer %d is quantised on the way in\n", path, why, layer);
        close(fd);
        return -2;
    }
    return fd;
}

int glm53f_i4file_open_layer(const Glm53fSt *st, const Glm53fCfg *c, int layer, const char *dir)
{
    uint8_t hdr[GLM53F_I4F_HEADER];
    int64_t slot = 0;
    return open_checked(st, c, layer, dir, &slot, hdr, 0);
}

int glm53f_i4file_verify_layer(const Glm53fSt *st, const Glm53fCfg *c, int layer, const char *dir)
{
    uint8_t hdr[GLM53F_I4F_HEADER];
    int64_t slot = 0;
    const int fd = open_checked(st, c, layer, dir, &slot, hdr, 0);
    if (fd < 0) return -1;
    uint8_t *buf = (uint8_t *)malloc((size_t)slot);
    if (!buf) { close(fd); return -1; }
    int bad = 0;
    for (int e = 0; e < c->n_experts; e++)
        if (pread(fd, buf, (size_t)slot, glm53f_i4file_offset(e, slot)) != (ssize_t)slot ||
            crc32_of(buf, (size_t)slot) != rd32(hdr + 48 + 4 * e))
            bad++;
    free(buf);
    close(fd);
    return bad;
}

static int read_at(int fd, void *buf, int64_t n, int64_t off)
{
    int64_t got = 0;
    while (got < n) {
        const ssize_t r = pread(fd, (char *)buf + got, (size_t)(n - got), off + got);
        if (r <= 0) return -1;
        got += r;
    }
    return 0;
}

/* One expert as a container slot: its FP8 matrices and scale grids read from the shards, the
 * device quantiser, the slot image back in img (zeroed padding). */
static int expert_slot(const Glm53fSt *st, const Glm53fCfg *c, int layer, int expert, uint8_t *host, uint8_t *dev,
                       uint8_t *slot_d, int64_t slot, uint8_t *img)
{
    const Glm53fTensor *t[6];
    if (expert_tensors(st, layer, expert, t)) return -1;
    int64_t qo[3], so[3];
    i4_slot(c, qo, so);
    if (g53h_memset(slot_d, 0, (size_t)slot)) return -1;
    for (int m = 0; m < 3; m++) {
        int rows, cols;
        mat_shape(c, m, &rows, &cols);
        const int br = c->fp8_block_r, bc = c->fp8_block_c;
        const int srows = (rows + br - 1) / br, scols = (cols + bc - 1) / bc;
        const int64_t wb = (int64_t)rows * cols, sb = (int64_t)srows * scols * 4;
        if (t[m]->nbytes != wb || t[3 + m]->nbytes != sb || t[3 + m]->dtype != GLM53F_DT_F32) return -1;
        if (read_at(st->fd[t[m]->shard], host, wb, t[m]->off) ||
            read_at(st->fd[t[3 + m]->shard], host + wb, sb, t[3 + m]->off))
            return -1;
        if (g53h_h2d(dev, host, (size_t)(wb + sb))) return -1;
        G53hMat src;
        memset(&src, 0, sizeof src);
        src.w = dev; src.s = (const float *)(dev + wb);
        src.rows = rows; src.cols = cols; src.br = br; src.bc = bc; src.scols = scols;
        if (g53h_i4_from_f8(slot_d + qo[m], (float *)(slot_d + so[m]), &src)) return -1;
    }
    return g53h_d2h(img, slot_d, (size_t)slot);
}

int glm53f_i4file_write_layer(const Glm53fSt *st, const Glm53fCfg *c, int layer, const char *dir)
{
    if (c->n_experts > (GLM53F_I4F_HEADER - 48) / 4) return -1;
    uint8_t hdr[GLM53F_I4F_HEADER];
    int64_t slot = 0;
    {
        const int fd = open_checked(st, c, layer, dir, &slot, hdr, 1);
        if (fd >= 0) { close(fd); return 1; }             /* already complete and valid */
    }
    uint64_t fp = 0;
    if (fingerprint(st, c, layer, &slot, &fp)) {
        fprintf(stderr, "glm53f: layer %d has no routed experts of one shape\n", layer);
        return -1;
    }
    for (int m = 0; m < 3; m++) {
        int rows, cols;
        mat_shape(c, m, &rows, &cols);
        if (cols % GLM53F_I4_GROUP) {
            fprintf(stderr, "glm53f: the int4 container needs columns a multiple of %d\n", GLM53F_I4_GROUP);
            return -1;
        }
    }
    char part[1024], path[1024];
    layer_path(part, sizeof part, dir, layer, ".part");
    layer_path(path, sizeof path, dir, layer, "");
    int64_t raw = 0;
    for (int m = 0; m < 3; m++) {
        int rows, cols;
        mat_shape(c, m, &rows, &cols);
        const int64_t r = (int64_t)rows * cols +
                          (int64_t)((rows + c->fp8_block_r - 1) / c->fp8_block_r) *
                              ((cols + c->fp8_block_c - 1) / c->fp8_block_c) * 4;
        if (r > raw) raw = r;
    }
    uint8_t *host = (uint8_t *)malloc((size_t)raw), *img = (uint8_t *)malloc((size_t)slot);
    uint8_t *dev = (uint8_t *)g53h_alloc((size_t)raw), *slot_d = (uint8_t *)g53h_alloc((size_t)slot);
    uint32_t *crc = (uint32_t *)calloc((size_t)c->n_experts, sizeof *crc);
    FILE *f = NULL;
    int ok = host && img && dev && slot_d && crc;
    if (ok && !(f = fopen(part, "wb"))) {
        fprintf(stderr, "glm53f: cannot create %s\n", part);
        ok = 0;
    }
    memset(hdr, 0, sizeof hdr);
    if (ok) ok = fwrite(hdr, 1, sizeof hdr, f) == sizeof hdr;          /* the header comes last */
    for (int e = 0; ok && e < c->n_experts; e++) {
        if (expert_slot(st, c, layer, e, host, dev, slot_d, slot, img)) {
            fprintf(stderr, "glm53f: layer %d expert %d could not be read\n", layer, e);
            ok = 0;
            break;
        }
        crc[e] = crc32_of(img, (size_t)slot);
        ok = fwrite(img, 1, (size_t)slot, f) == (size_t)slot;
        if (!ok) fprintf(stderr, "glm53f: writing %s failed (disk full?)\n", part);
    }
    if (f && fclose(f)) ok = 0;
    if (ok) {
        memcpy(hdr, I4F_MAGIC, 8);
        le32(hdr + 8, I4F_VERSION);
        le32(hdr + 12, (uint32_t)layer);
        le32(hdr + 16, (uint32_t)c->n_experts);
        le32(hdr + 20, GLM53F_I4_GROUP);
        le64(hdr + 24, (uint64_t)slot);
        le64(hdr + 32, fp);
        le32(hdr + 40, 1);
        for (int e = 0; e < c->n_experts; e++) le32(hdr + 48 + 4 * e, crc[e]);
        FILE *h = fopen(part, "r+b");
        ok = h && fwrite(hdr, 1, sizeof hdr, h) == sizeof hdr;
        if (h && fclose(h)) ok = 0;
    }
    if (ok) {
        remove(path);
        if (rename(part, path)) {
            fprintf(stderr, "glm53f: cannot rename %s\n", part);
            ok = 0;
        }
    }
    if (!ok) remove(part);
    free(host);
    free(img);
    free(crc);
    if (dev) g53h_free(dev);
    if (slot_d) g53h_free(slot_d);
    return ok ? 0 : -1;
}
