/* g53h_ckpt.c - routed experts read from the checkpoint for the HBM expert cache.
 *
 * Two parts:
 *   - g53h_st_open/close/index: this library's reader of the safetensors shards into the
 *     reference's index type (include/glm53f_st.h, src/io/glm53f_st.h:24-58). Each shard is
 *     [8-byte little-endian header length N][N bytes of JSON][data]; a header entry
 *     "name": {"dtype": "F8_E4M3", "shape": [r, c], "data_offsets": [a, b]} places the tensor
 *     at absolute offset 8 + N + a of its shard. The JSON parser below reads exactly that
 *     grammar (objects, arrays, strings, numbers; "__metadata__" skipped).
 *   - G53hCkpt: the expert store of glm53f_cache_init over any Glm53fSt (this reader's or the
 *     reference's). At init it scans t[] once and files the six tensors of every routed expert
 *     (src/io/glm53f_load.c:11 names them "model.language_model.layers.L.mlp.experts.E.
 *     {gate,up,down}_proj.{weight,weight_scale_inv}") in a direct table indexed by
 *     (layer, expert, tensor), so a fetch is six array reads, no name formatting or hashing.
 *     A fetch reads the expert into one of a few pinned staging buffers: the three weights in
 *     one read and the three scale grids in another when each set is one run in one shard
 *     (how the released checkpoint is laid out, src/io/glm53f_load.c:66-101), else one read
 *     per tensor. With an O_DIRECT descriptor (dfd >= 0) the weight run is read through it,
 *     widened to GLM53F_ST_ALIGN boundaries, which keeps a streamed expert out of the host's
 *     page cache (src/io/glm53f_st.h:60-75). The buffer stays busy until the cache reports the
 *     copy to HBM complete (done). */
#define _GNU_SOURCE
#include <dirent.h>
#include <errno.h>
#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include "g53h.h"
#include "g53h_ckpt.h"
#include "glm53f.h"
#include "glm53f_st.h"

/* ------------------------------------------------------------------ JSON ---- */
typedef struct {
    const char *p, *end;
    int bad;
} Js;

static void js_ws(Js *j)
{
    while (j->p < j->end && (*j->p == ' ' || *j->p == '\n' || *j->p == '\r' || *j->p == '\t')) j->p++;
}

static int js_eat(Js *j, char ch)
{
    js_ws(j);
    if (j->p < j->end && *j->p == ch) { j->p++; return 1; }
    return 0;
}

/* A string into out (escapes kept as the escaped character; names are plain ASCII). */
static int js_str(Js *j, char *out, size_t cap)
{
    js_ws(j);
    if (j->p >= j->end || *j->p != '"') { j->bad = 1; return -1; }
    j->p++;
    size_t n = 0;
    while (j->p < j->end && *j->p != '"') {
        char ch = *j->p++;
        if (ch == '\\' && j->p < j->end) ch = *j->p++;
        if (n + 1 < cap) out[n++] = ch;
        else j->bad = 1;
    }
    if (j->p >= j->end) { j->bad = 1; return -1; }
    j->p++;
    out[n] = 0;
    return (int)n;
}

static int64_t js_int(Js *j)
{
    /* parsed by hand within [p, end): the header buffer is not NUL-terminated */
    js_ws(j);
    const char *q = j->p;
    const int neg = q < j->end && *q == '-';
    if (neg) q++;
    if (q >= j->end || *q < '0' || *q > '9') { j->bad = 1; return 0; }
    uint64_t v = 0;
    for (; q < j->end && *q >= '0' && *q <= '9'; q++) {
        if (v > (UINT64_C(1) << 62) / 10) { j->bad = 1; return 0; }
        v = v * 10 + (uint64_t)(*q - '0');
    }
    j->p = q;
    return neg ? -(int64_t)v : (int64_t)v;
}

/* Skip any value. */
static void js_skip(Js *j)
{
    js_ws(j);
    if (j->p >= j->end) { j->bad = 1; return; }
    const char ch = *j->p;
    if (ch == '"') {
        j->p++;
        while (j->p < j->end && *j->p != '"') j->p += (*j->p == '\\' && j->end - j->p > 1) ? 2 : 1;
        if (j->p >= j->end) { j->bad = 1; return; }
        j->p++;
    } else if (ch == '{' || ch == '[') {
        const char close = ch == '{' ? '}' : ']';
        j->p++;
        if (js_eat(j, close)) return;
        do {
            if (ch == '{') { char k[256]; js_str(j, k, sizeof k); if (!js_eat(j, ':')) { j->bad = 1; return; } }
            js_skip(j);
        } while (!j->bad && js_eat(j, ','));
        if (!js_eat(j, close)) j->bad = 1;
    } else {
        while (j->p < j->end && *j->p != ',' && *j->p != '}' && *j->p != ']') j->p++;
    }
}

static Glm53fDtype dtype_of(const char *s)
{
    if (!strcmp(s, "F8_E4M3")) return GLM53F_DT_F8_E4M3;
    if (!strcmp(s, "BF16")) return GLM53F_DT_BF16;
    if (!strcmp(s, "F16")) return GLM53F_DT_F16;
    if (!strcmp(s, "F32")) return GLM53F_DT_F32;
    if (!strcmp(s, "U8")) return GLM53F_DT_U8;
    return GLM53F_DT_UNKNOWN;
}

static char *pool_add(Glm53fSt *s, const char *name)
{
    const size_t n = strlen(name) + 1;
    if (s->strlen_ + n > s->strcap) {
        /* names are referenced by pointer: grow by chaining a fresh block, never by realloc */
        const size_t cap = n > (1u << 20) ? n : (1u << 20);
        char *blk = (char *)malloc(cap + sizeof(char *));
        if (!blk) return NULL;
        *(char **)blk = s->strpool;              /* previous block, freed at close */
        s->strpool = blk;
        s->strcap = cap;
        s->strlen_ = 0;
    }
    char *d = s->strpool + sizeof(char *) + s->strlen_;
    memcpy(d, name, n);
    s->strlen_ += n;
    return d;
}

/* Index one shard's header. */
static int index_shard(Glm53fSt *s, int shard, const char *path)
{
    uint8_t lenb[8];
    if (pread(s->fd[shard], lenb, 8, 0) != 8) { fprintf(stderr, "g53h_st_open: %s: short header\n", path); return -1; }
    uint64_t n = 0;
    for (int i = 7; i >= 0; i--) n = (n << 8) | lenb[i];
    struct stat stt;
    if (fstat(s->fd[shard], &stt) != 0 || n == 0 || n > (uint64_t)stt.st_size - 8 || n > (1ull << 31)) {
        fprintf(stderr, "g53h_st_open: %s: bad header length %llu\n", path, (unsigned long long)n);
        return -1;
    }
    char *h = (char *)malloc(n);
    if (!h || pread(s->fd[shard], h, n, 8) != (ssize_t)n) {
        free(h);
        fprintf(stderr, "g53h_st_open: %s: cannot read the header\n", path);
        return -1;
    }
    Js j = {h, h + n, 0};
    int rc = 0;
    if (!js_eat(&j, '{')) rc = -1;
    if (!rc && !js_eat(&j, '}')) {
        do {
            char name[512];
            if (js_str(&j, name, sizeof name) < 0 || !js_eat(&j, ':')) { rc = -1; break; }
            if (!strcmp(name, "__metadata__")) { js_skip(&j); continue; }
            Glm53fTensor t;
            memset(&t, 0, sizeof t);
            int64_t a = -1, b = -1;
            if (!js_eat(&j, '{')) { rc = -1; break; }
            if (!js_eat(&j, '}')) {
                do {
                    char key[64];
                    if (js_str(&j, key, sizeof key) < 0 || !js_eat(&j, ':')) { rc = -1; break; }
                    if (!strcmp(key, "dtype")) {
                        char dt[32];
                        js_str(&j, dt, sizeof dt);
                        t.dtype = dtype_of(dt);
                    } else if (!strcmp(key, "shape")) {
                        if (!js_eat(&j, '[')) { rc = -1; break; }
                        if (!js_eat(&j, ']')) {
                            do {
                                const int64_t v = js_int(&j);
                                if (t.ndim < 8) t.shape[t.ndim] = v;
                                t.ndim++;
                            } while (js_eat(&j, ','));
                            if (!js_eat(&j, ']')) { rc = -1; break; }
                        }
                    } else if (!strcmp(key, "data_offsets")) {
                        if (!js_eat(&j, '[')) { rc = -1; break; }
                        a = js_int(&j);
                        if (!js_eat(&j, ',')) { rc = -1; break; }
                        b = js_int(&j);
                        if (!js_eat(&j, ']')) { rc = -1; break; }
                    } else {
                        js_skip(&j);
                    }
                } while (!j.bad && js_eat(&j, ','));
                if (rc || !js_eat(&j, '}')) { rc = -1; break; }
            }
            if (j.bad || a < 0 || b < a || t.ndim > 8 || (uint64_t)b > (uint64_t)stt.st_size - 8 - n) {
                fprintf(stderr, "g53h_st_open: %s: bad entry %s\n", path, name);
                rc = -1;
                break;
            }
            t.shard = shard;
            t.off = (int64_t)(8 + n) + a;
            t.nbytes = b - a;
            t.name = pool_add(s, name);
            if (!t.name) { rc = -1; break; }
            if (s->nt % 1024 == 0) {
                Glm53fTensor *nt = (Glm53fTensor *)realloc(s->t, (size_t)(s->nt + 1024) * sizeof *nt);
                if (!nt) { rc = -1; break; }
                s->t = nt;
            }
            s->t[s->nt++] = t;
        } while (!j.bad && js_eat(&j, ','));
        if (!rc && !js_eat(&j, '}')) rc = -1;
    }
    if (rc || j.bad) fprintf(stderr, "g53h_st_open: %s: malformed header\n", path);
    free(h);
    return rc || j.bad ? -1 : 0;
}

static int cmp_str(const void *a, const void *b) { return strcmp(*(char *const *)a, *(char *const *)b); }

int g53h_st_open(Glm53fSt *s, const char *dir, int direct)
{
    memset(s, 0, sizeof *s);
    DIR *d = opendir(dir);
    if (!d) { fprintf(stderr, "g53h_st_open: cannot open %s\n", dir); return -1; }
    char **names = NULL;
    int n = 0, cap = 0;
    struct dirent *e;
    while ((e = readdir(d)) != NULL) {
        const size_t l = strlen(e->d_name);
        if (l < 12 || strcmp(e->d_name + l - 12, ".safetensors")) continue;
        if (n == cap) {
            cap = cap ? 2 * cap : 64;
            char **nn = (char **)realloc(names, (size_t)cap * sizeof *nn);
            if (!nn) break;
            names = nn;
        }
        names[n++] = strdup(e->d_name);
    }
    closedir(d);
    if (!n) { fprintf(stderr, "g53h_st_open: no .safetensors in %s\n", dir); free(names); return -1; }
    qsort(names, (size_t)n, sizeof *names, cmp_str);
    s->fd = (int *)malloc((size_t)n * sizeof(int));
    s->dfd = (int *)malloc((size_t)n * sizeof(int));
    s->path = (char **)calloc((size_t)n, sizeof(char *));
    int rc = s->fd && s->dfd && s->path ? 0 : -1;
    for (int i = 0; i < n; i++) {
        if (s->fd) s->fd[i] = -1;
        if (s->dfd) s->dfd[i] = -1;
    }
    for (int i = 0; i < n && !rc; i++) {
        const size_t l = strlen(dir) + strlen(names[i]) + 2;
        s->path[i] = (char *)malloc(l);
        snprintf(s->path[i], l, "%s/%s", dir, names[i]);
        s->nshard = i + 1;
        s->fd[i] = open(s->path[i], O_RDONLY);
        if (s->fd[i] < 0) { fprintf(stderr, "g53h_st_open: cannot open %s\n", s->path[i]); rc = -1; break; }
        if (direct) s->dfd[i] = open(s->path[i], O_RDONLY | O_DIRECT);
        rc = index_shard(s, i, s->path[i]);
    }
    for (int i = 0; i < n; i++) free(names[i]);
    free(names);
    if (rc) g53h_st_close(s);
    return rc;
}

void g53h_st_close(Glm53fSt *s)
{
    for (int i = 0; i < s->nshard; i++) {
        if (s->fd && s->fd[i] >= 0) close(s->fd[i]);
        if (s->dfd && s->dfd[i] >= 0) close(s->dfd[i]);
        if (s->path) free(s->path[i]);
    }
    free(s->fd);
    free(s->dfd);
    free(s->path);
    free(s->t);
    char *blk = s->strpool;
    while (blk) {
        char *prev = *(char **)blk;
        free(blk);
        blk = prev;
    }
    memset(s, 0, sizeof *s);
}

int g53h_st_index(const Glm53fSt *s, const char *name)
{
    for (int i = 0; i < s->nt; i++)
        if (s->t[i].name && !strcmp(s->t[i].name, name)) return i;
    return -1;
}

/* ------------------------------------------------------------ expert store ---- */
#define NT 6                            /* gate, up, down weights; gate, up, down scales */

struct G53hCkpt {
    const Glm53fSt *st;
    int n_layers, n_experts, br, bc;
    int rows[3], cols[3];
    int32_t *tab;                       /* [n_layers][n_experts][NT] -> index into st->t, -1 */
    int nstage;
    uint8_t **stage;                    /* pinned buffers                               */
    int32_t *stage_key;                 /* expert key held, -1 free                     */
    size_t stage_bytes, warea;          /* buffer size; weight area (then the scales)   */
};

static int64_t al_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

/* "model.language_model.layers.L.mlp.experts.E.P_proj.K" -> (L, E, tensor), or -1. */
static int parse_expert_name(const char *name, int *layer, int *expert)
{
    static const char pre[] = "model.language_model.layers.";
    if (strncmp(name, pre, sizeof pre - 1)) return -1;
    const char *p = name + sizeof pre - 1;
    char *e;
    const long L = strtol(p, &e, 10);
    if (e == p || strncmp(e, ".mlp.experts.", 13)) return -1;
    p = e + 13;
    const long E = strtol(p, &e, 10);
    if (e == p || *e != '.') return -1;
    p = e + 1;
    int m;
    if (!strncmp(p, "gate_proj.", 10)) m = 0;
    else if (!strncmp(p, "up_proj.", 8)) m = 1;
    else if (!strncmp(p, "down_proj.", 10)) m = 2;
    else return -1;
    p = strchr(p, '.') + 1;
    int k;
    if (!strcmp(p, "weight")) k = m;
    else if (!strcmp(p, "weight_scale_inv")) k = 3 + m;
    else return -1;
    *layer = (int)L;
    *expert = (int)E;
    return k;
}

/* Matrix shapes, block sizes and the staging layout from the config. */
static int ckpt_geometry(G53hCkpt *k, const Glm53fCfg *cfg)
{
    k->n_experts = cfg->n_experts;
    k->br = cfg->fp8_block_r;
    k->bc = cfg->fp8_block_c;
    k->rows[0] = k->rows[1] = cfg->moe_inter; k->cols[0] = k->cols[1] = cfg->hidden;
    k->rows[2] = cfg->hidden; k->cols[2] = cfg->moe_inter;
    if (k->br < 1 || k->bc < 1 || k->n_experts < 1 || cfg->hidden < 1 || cfg->moe_inter < 1) return -1;
    int64_t wb = 0, sb = 0;
    for (int m = 0; m < 3; m++) {
        wb += (int64_t)k->rows[m] * k->cols[m];
        sb += (int64_t)((k->rows[m] + k->br - 1) / k->br) * ((k->cols[m] + k->bc - 1) / k->bc) * 4;
    }
    k->warea = (size_t)al_up(wb + 2 * GLM53F_ST_ALIGN, GLM53F_ST_ALIGN);
    k->stage_bytes = (size_t)al_up((int64_t)k->warea + sb, GLM53F_ST_ALIGN);
    return 0;
}

G53hCkpt *g53h_ckpt_new(const Glm53fSt *st, const Glm53fCfg *cfg, int n_layers, int nstage)
{
    if (!st || !st->t || !cfg || n_layers <= 0 || nstage < 0) return NULL;
    G53hCkpt *k = (G53hCkpt *)calloc(1, sizeof *k);
    if (!k) return NULL;
    k->st = st;
    k->n_layers = n_layers;
    if (ckpt_geometry(k, cfg)) { free(k); return NULL; }
    const size_t ntab = (size_t)n_layers * k->n_experts * NT;
    k->tab = (int32_t *)malloc(ntab * sizeof(int32_t));
    if (!k->tab) { g53h_ckpt_free(k); return NULL; }
    for (size_t i = 0; i < ntab; i++) k->tab[i] = -1;
    for (int i = 0; i < st->nt; i++) {
        int L, E;
        const int t = st->t[i].name ? parse_expert_name(st->t[i].name, &L, &E) : -1;
        if (t < 0 || L < 0 || L >= n_layers || E < 0 || E >= k->n_experts) continue;
        k->tab[((size_t)L * k->n_experts + E) * NT + t] = i;
    }
    k->nstage = nstage;
    if (!nstage) return k;
    k->stage = (uint8_t **)calloc((size_t)nstage, sizeof(uint8_t *));
    k->stage_key = (int32_t *)malloc((size_t)nstage * sizeof(int32_t));
    if (!k->stage || !k->stage_key) { g53h_ckpt_free(k); return NULL; }
    for (int i = 0; i < nstage; i++) {
        k->stage_key[i] = -1;
        k->stage[i] = (uint8_t *)g53h_host_alloc(k->stage_bytes);
        if (!k->stage[i]) { g53h_ckpt_free(k); return NULL; }
    }
    return k;
}

void g53h_ckpt_free(G53hCkpt *k)
{
    if (!k) return;
    for (int i = 0; k->stage && i < k->nstage; i++)
        if (k->stage[i]) g53h_host_free(k->stage[i]);
    free(k->stage);
    free(k->stage_key);
    free(k->tab);
    free(k);
}

static int read_full(int fd, void *buf, size_t n, int64_t off)
{
    size_t got = 0;
    while (got < n) {
        const ssize_t r = pread(fd, (char *)buf + got, n - got, (off_t)(off + (int64_t)got));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return -1;
        got += (size_t)r;
    }
    return 0;
}

/* Read [off, off + n) of a shard through its O_DIRECT descriptor into buf (aligned, at least
 * n + 2 * GLM53F_ST_ALIGN long); *lead receives where the payload starts in buf. */
static int read_direct(int dfd, uint8_t *buf, int64_t off, int64_t n, int64_t *lead)
{
    const int64_t a0 = off / GLM53F_ST_ALIGN * GLM53F_ST_ALIGN, a1 = al_up(off + n, GLM53F_ST_ALIGN);
    *lead = off - a0;
    int64_t got = 0;
    while (got < a1 - a0) {
        const ssize_t r = pread(dfd, buf + got, (size_t)(a1 - a0 - got), (off_t)(a0 + got));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) break;                              /* end of file inside the window */
        got += r;
        if (r % GLM53F_ST_ALIGN) break;
    }
    return got >= *lead + n ? 0 : -1;
}

/* Validate and read expert (layer, expert) into buf (k->stage_bytes long) and point q at it. */
static int ckpt_read(const G53hCkpt *k, int layer, int expert, uint8_t *buf, Glm53fExpertQ *q)
{
    if (layer < 0 || layer >= k->n_layers || expert < 0 || expert >= k->n_experts) return -1;
    const int32_t *ix = k->tab + ((size_t)layer * k->n_experts + expert) * NT;
    const Glm53fSt *st = k->st;
    const Glm53fTensor *t[NT];
    for (int i = 0; i < NT; i++) {
        if (ix[i] < 0) {
            fprintf(stderr, "glm53f_cache: L%d expert %d: %s tensor missing from the checkpoint\n", layer, expert,
                    i < 3 ? "a weight" : "a scale");
            return -1;
        }
        t[i] = &st->t[ix[i]];
    }
    for (int m = 0; m < 3; m++) {
        const int sr = (k->rows[m] + k->br - 1) / k->br, sc = (k->cols[m] + k->bc - 1) / k->bc;
        if (t[m]->dtype != GLM53F_DT_F8_E4M3 || t[m]->ndim != 2 || t[m]->shape[0] != k->rows[m] ||
            t[m]->shape[1] != k->cols[m] || t[m]->nbytes != (int64_t)k->rows[m] * k->cols[m] ||
            t[3 + m]->dtype != GLM53F_DT_F32 || t[3 + m]->ndim != 2 || t[3 + m]->shape[0] != sr ||
            t[3 + m]->shape[1] != sc || t[3 + m]->nbytes != (int64_t)sr * sc * 4) {
            fprintf(stderr, "glm53f_cache: L%d expert %d matrix %d is not FP8 [%d,%d] with an F32 [%d,%d] scale grid\n",
                    layer, expert, m, k->rows[m], k->cols[m], sr, sc);
            return -1;
        }
    }
    /* weights: one run when the three lie back to back in one shard */
    int64_t wlo = t[0]->off, whi = 0, wsum = 0, slo = t[3]->off, shi = 0, ssum = 0;
    int one = 1;
    for (int m = 0; m < 3; m++) {
        one &= t[m]->shard == t[0]->shard && t[3 + m]->shard == t[0]->shard;
        if (t[m]->off < wlo) wlo = t[m]->off;
        if (t[m]->off + t[m]->nbytes > whi) whi = t[m]->off + t[m]->nbytes;
        wsum += t[m]->nbytes;
        if (t[3 + m]->off < slo) slo = t[3 + m]->off;
        if (t[3 + m]->off + t[3 + m]->nbytes > shi) shi = t[3 + m]->off + t[3 + m]->nbytes;
        ssum += t[3 + m]->nbytes;
    }
    const int wrun = one && whi - wlo == wsum, srun = one && shi - slo == ssum;
    const uint8_t *w[3];
    const float *s[3];
    if (wrun) {
        const int sh = t[0]->shard;
        int64_t lead = 0;
        const int dfd = st->dfd ? st->dfd[sh] : -1;
        if (dfd >= 0 && read_direct(dfd, buf, wlo, wsum, &lead) == 0) {
            /* read through O_DIRECT */
        } else {
            lead = 0;
            if (read_full(st->fd[sh], buf, (size_t)wsum, wlo)) goto fail;
        }
        for (int m = 0; m < 3; m++) w[m] = buf + lead + (t[m]->off - wlo);
    } else {
        int64_t o = 0;
        for (int m = 0; m < 3; m++) {
            if (read_full(st->fd[t[m]->shard], buf + o, (size_t)t[m]->nbytes, t[m]->off)) goto fail;
            w[m] = buf + o;
            o += t[m]->nbytes;
        }
    }
    uint8_t *sbuf = buf + k->warea;
    if (srun) {
        if (read_full(st->fd[t[3]->shard], sbuf, (size_t)ssum, slo)) goto fail;
        for (int m = 0; m < 3; m++) s[m] = (const float *)(sbuf + (t[3 + m]->off - slo));
    } else {
        int64_t o = 0;
        for (int m = 0; m < 3; m++) {
            if (read_full(st->fd[t[3 + m]->shard], sbuf + o, (size_t)t[3 + m]->nbytes, t[3 + m]->off)) goto fail;
            s[m] = (const float *)(sbuf + o);
            o += t[3 + m]->nbytes;
        }
    }
    Glm53fMat *out[3] = {&q->gate, &q->up, &q->down};
    for (int m = 0; m < 3; m++) {
        memset(out[m], 0, sizeof *out[m]);
        out[m]->w = w[m];
        out[m]->s = s[m];
        out[m]->dt = GLM53F_WF8;
        out[m]->rows = k->rows[m];
        out[m]->cols = k->cols[m];
        out[m]->br = k->br;
        out[m]->bc = k->bc;
        out[m]->scols = (k->cols[m] + k->bc - 1) / k->bc;
    }
    return 0;
fail:
    fprintf(stderr, "glm53f_cache: short read of L%d expert %d from the checkpoint\n", layer, expert);
    return -1;
}

int g53h_ckpt_view(G53hCkpt *k, int layer, int expert, Glm53fExpertQ *q)
{
    int b = -1;
    for (int i = 0; i < k->nstage; i++)
        if (k->stage_key[i] < 0) { b = i; break; }
    if (b < 0) return G53H_CKPT_BUSY;
    const int rc = ckpt_read(k, layer, expert, k->stage[b], q);
    if (rc == 0) k->stage_key[b] = layer * k->n_experts + expert;
    return rc;
}

size_t g53h_st_expert_bytes(const Glm53fCfg *cfg)
{
    G53hCkpt k;
    memset(&k, 0, sizeof k);
    if (ckpt_geometry(&k, cfg)) return 0;
    return k.stage_bytes;
}

int g53h_st_read_expert(const Glm53fSt *st, const Glm53fCfg *cfg, int layer, int expert, void *buf, size_t cap,
                        Glm53fExpertQ *q)
{
    if (cap < g53h_st_expert_bytes(cfg)) return -1;
    G53hCkpt *k = g53h_ckpt_new(st, cfg, layer + 1, 0);
    if (!k) return -1;
    const int rc = ckpt_read(k, layer, expert, (uint8_t *)buf, q);
    g53h_ckpt_free(k);
    return rc;
}

void g53h_ckpt_done(G53hCkpt *k, int layer, int expert)
{
    const int32_t key = layer * k->n_experts + expert;
    for (int i = 0; i < k->nstage; i++)
        if (k->stage_key[i] == key) { k->stage_key[i] = -1; return; }
}
