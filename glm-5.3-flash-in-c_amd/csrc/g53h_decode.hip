/* g53h_decode.hip - single-token decode of one MoE layer in one launch (k_dec_layer).
 *
 * The layer (reference src/core/glm53f_ops.c:1144-1342 at T = 1, with the router of
 * :945-976) is cut into work items of one 8 KB step of HBM codes for one wave:
 *
 *   R   one router row (bf16, 8 KB): the score of one expert
 *   G   one (gate row o, up row o) pair of one slot (2 x 4 KB of E4M3 codes) and its SwiGLU
 *   A   half of one slot's activation vector, copied into LDS
 *   D   four down rows of one slot (4 x 2 KB of codes): four contributions
 *
 * One workgroup of 12 waves per CU. Every workgroup owns the same share of every slot's gate/up
 * rows and of every slot's down rows, so the final weighted combine of its rows is local to
 * it. Its list: its router rows; its shared-expert G items; the shared expert's A and D
 * items; its G items of every routed slot, slot by slot; then per routed slot its A and D
 * items. The waves take items from the list through an LDS counter, one ahead: the codes of
 * the next item are in flight while the current one is multiplied.
 *
 * Codes are read coalesced (each load instruction of a wave covers consecutive bytes) and
 * the lanes trade 16-byte chunks through LDS so that each holds one 128-column block, the
 * unit of the reference's arithmetic.
 *
 * Two things cross workgroups, both through words tagged with the launch's epoch in their
 * upper half and published by atomic exchange (performed past the writer's L2); readers load
 * them coherently and re-read until the tags are current, so nothing is ever cleared and no
 * intra-launch barrier is needed:
 *   - the scores: the last wave of every workgroup waits for all of them, selects the top-k,
 *     and loads the chosen experts' descriptors; meanwhile only a few waves stream (the
 *     shared expert), so that the routing's loads are not queued behind a saturated memory
 *     system, and the other waves start the routed slots when it is done;
 *   - the activations: a slot's A items read what every workgroup's G items wrote, long
 *     after they were written in the normal case.
 *
 * Arithmetic is the reference's, bit for bit (see g53h_gemv.h). Every wait is bounded: a wait
 * that runs out sets an error flag (read by g53h_decode_errors) and the wave goes on, so the
 * grid always drains. The grid is one workgroup per CU, all resident at once.
 */
#include <hip/hip_runtime.h>
#include <math.h>

#include "g53h.h"
#include "g53h_core.h"
#include "g53h_gemv.h"
#include "g53h_kern.h"
#include "g53h_runtime.h"
#include "g53h_xwg.h"

#define G53_DEC_RPD 4              /* down rows per item                                 */
#define G53_DEC_NGRP (G53_DEC_E / G53_DEC_RPD)
#define G53_DEC_MAXRG 4            /* row groups one workgroup owns (grid >= 256)         */
#define G53_DEC_NT 768             /* threads of a k_dec_layer workgroup (one per CU)     */
#define G53_DEC_DTAB ((G53_DEC_NT / 64 - 1 - G53_DEC_EARLY) * 8192)   /* staging bytes */
#ifndef G53_DEC_EARLY
#define G53_DEC_EARLY 3            /* waves that stream before the routing is known       */
#endif
#define G53_DEC_NENT 3             /* activation copies a workgroup keeps in LDS          */
#define G53_DEC_ROT 16             /* copies of the tagged activations, used in rotation  */
/* The sum, in lane order, of the doubles held by lanes base .. base+N-1 (base = lane rounded
 * down to a multiple of N), valid in lane base: the reference's sequential sum over a row's
 * blocks. The terms pass through pt, 64 doubles of LDS private to the wave. */
template <int N>
__device__ __forceinline__ double g53_row_sum(double t, double *pt, int lane)
{
    pt[lane] = t;
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    double s = 0.0;
    if ((lane & (N - 1)) == 0) {
#pragma unroll
        for (int k = 0; k < N; k += 2) {
            const double2 q = *(const double2 *)(pt + lane + k);
            s = s + q.x;
            s = s + q.y;
        }
    }
    __builtin_amdgcn_wave_barrier();
    return s;
}

/* One gate/up row pair (lanes 0-31 gate blocks, 32-63 up blocks) with x in LDS: the two row
 * sums in block order and the SwiGLU, valid in lane 0. */
__device__ __forceinline__ float g53_gateup_pair(const g53_u4 (&c)[8], float sc, const float *xs, double *pt,
                                                 float limit, const uint64_t *etab, int lane)
{
    const int bb = lane & 31;
    const double t = g53_blk_pad(c, xs + bb * G53_PADB) * (double)sc;
    const float v = (float)g53_row_sum<32>(t, pt, lane);
    const float u = __shfl(v, 32);
    return g53_swiglu1_tab(v, u, limit, etab);
}


/* Diagnostics: per-workgroup timestamps (100 MHz) into a.trace when it is set. */
#define G53_TRACE(k) do { if (a.trace && lane == 0) \
    a.trace[(size_t)blockIdx.x * 32 + (k)] = __builtin_amdgcn_s_memrealtime(); } while (0)


/* --------------------------------------------------------------- k_dec_layer ---- */
struct G53LayerArgs {
    float *out;
    const float *x;
    const uint16_t *router;        /* bf16 [NE][E]                                       */
    const float *bias;
    const G53hExpert *experts;
    const G53hExpert *shared;
    g53_u64 *score;                /* [NE] tagged scores                                 */
    g53_u64 *act;                  /* [MAXK + 1][I] tagged activations, slot K = shared  */
    int *err;
    int *idx_out;                  /* the routing for the caller (may be NULL)            */
    float *w_out;
    int NE, K, norm_topk;
    unsigned epoch;
    float routed_scale, limit;
    int spin;                      /* polls before a wait on another workgroup gives up */
    g53_u64 *trace;                /* optional: [grid][32] timestamps and counters       */
};

enum { G53_IT_NONE = 0, G53_IT_R = 1, G53_IT_G = 2, G53_IT_D = 3, G53_IT_A = 4 };

struct G53Item {
    int kind, s, r;                /* slot (K = the shared expert), and row / o / group / half */
    int t;                         /* position of the slot in the down phase (0 = shared) */
};

/* The workgroup's list (workgroup b of G, one per CU):
 *   R      router rows b, b + G, ... (score of one expert each), taken by the first waves
 *          before the list starts
 *   S      gate/up rows [g_lo, g_lo + g_n) of the shared expert (G items of slot K)
 *   G      gate/up rows [g_lo, g_lo + g_n) of every routed slot, slot by slot
 *   A, D   per slot (the shared expert first, then the routed slots in top-k order): the two
 *          halves of its activation vector (A, into LDS entry t % NENT) and its down row
 *          groups [rg_lo, rg_lo + n_rg) (D), a slot's A items one slot ahead of its D items
 * Its waves take items in this order through an LDS counter. The last wave first computes
 * the routing (the top-k, once the scores of every workgroup are in, and the chosen
 * experts' descriptors), the one dependency on other workgroups at the start; a few waves
 * meanwhile keep the memory busy with the shared expert's rows. By the time a workgroup
 * reaches a slot's A items, every workgroup has long finished that slot's gate/up rows. */
struct G53List {
    int nR, g_lo, g_n, rg_lo, n_rg, K, hs, i_s, i_sd, i_g, n;
};

__device__ __forceinline__ G53Item g53_item(const G53List &l, int i, int b, int G)
{
    G53Item it{G53_IT_NONE, 0, 0, 0};
    if (i < l.i_sd) { it.kind = G53_IT_G; it.s = l.K; it.t = 0; it.r = l.g_lo + i - l.i_s; return it; }
    if (i < l.i_g) {
        const int j = i - l.i_sd;
        it.kind = G53_IT_G; it.s = j / l.g_n; it.t = it.s + l.hs; it.r = l.g_lo + j % l.g_n;
        return it;
    }
    if (i < l.n) {
        /* the down phase, slot by slot in time order t (t = 0 the shared expert when there is
         * one): A(0) A(0), then A(t) A(t) D(t-1)... for t = 1 .. T-1, then D(T-1)...; a slot's
         * activations are copied one slot ahead of its down rows */
        const int T = l.K + l.hs, per = 2 + l.n_rg;
        int j = i - l.i_g, t, q;
        if (j < 2) { t = 0; q = j; }
        else { j -= 2; const int k = j / per + 1; q = j % per; if (k < T) { t = q < 2 ? k : k - 1; } else { t = T - 1; q += 2; } }
        it.t = t;
        it.s = l.hs ? (t == 0 ? l.K : t - 1) : t;
        if (q < 2) { it.kind = G53_IT_A; it.r = q; } else { it.kind = G53_IT_D; it.r = l.rg_lo + q - 2; }
    }
    return it;
}

/* Addresses of one item's loads and this lane's block scale. Codes are read coalesced: load k
 * of lane l reads 16 bytes at p + k * stride, so each load instruction of the wave covers
 * consecutive HBM bytes (a G item: 512 bytes of the gate row from lanes 0-31 and 512 of the
 * up row from lanes 32-63, stride 512; a D item: 1 KB of its four consecutive rows, stride
 * 1024), and the lanes then trade 16-byte chunks through LDS so that each holds the 128
 * bytes of its own block (g53_xpose). A and R items read 128 consecutive bytes per lane
 * (stride 16).
 * Items that read nothing point at the input vector instead, so that the loop issues its
 * loads from one place with no branch around them (a branch makes the compiler wait for the
 * loads where the paths join). Returns whether the item's codes are real. The matrices have
 * 128 x 128 blocks, so the scale row of output row r is r >> 7. */
__device__ __forceinline__ bool g53_addr(const G53Item &it, const G53hExpert *st, const g53_u64 *act,
                                         const uint16_t *router, const float *dummy, int lane, const uint8_t *&p,
                                         const float *&ps, int &stride)
{
    p = (const uint8_t *)dummy + lane * 128;
    ps = dummy;
    stride = 16;
    if (it.kind == G53_IT_A) {                /* 16 tagged activations per lane */
        p = (const uint8_t *)(act + (size_t)it.s * G53_DEC_I + it.r * 1024 + lane * 16);
        return true;
    }
    if (it.kind == G53_IT_G) {
        const G53hExpert &ex = st[it.s];
        if (!ex.gate.w) return false;
        const G53hMat &m = lane < 32 ? ex.gate : ex.up;
        const int b = lane & 31;
        p = m.w + (size_t)it.r * G53_DEC_E + b * 16;
        ps = m.s + (size_t)(it.r >> 7) * m.scols + b;
        stride = 512;
        return true;
    }
    if (it.kind == G53_IT_D) {
        const G53hExpert &ex = st[it.s];
        if (!ex.gate.w) return false;
        const G53hMat &m = ex.down;
        const int b = lane & 15, d = it.r * G53_DEC_RPD + (lane >> 4);
        p = m.w + (size_t)it.r * G53_DEC_RPD * G53_DEC_I + lane * 16;
        ps = m.s + (size_t)(d >> 7) * m.scols + b;
        stride = 1024;
        return true;
    }
    return false;
}

/* A use of every register of a code buffer: the compiler then waits for the buffer's loads
 * here on every path, so that no load into the buffer is still outstanding when the next one
 * is issued into it (which would otherwise make that issue wait for the other buffer's loads
 * too, loads completing in order). */
__device__ __forceinline__ void g53_touch(const g53_u4 (&c)[8], float sc)
{
#pragma unroll
    for (int k = 0; k < 8; k++) asm volatile("" ::"v"(c[k]));
    asm volatile("" ::"v"(sc));
}

#if defined(__HIP_DEVICE_COMPILE__)
typedef __attribute__((address_space(1))) const g53_u4 g53_gv4;
#else
typedef const g53_u4 g53_gv4;
#endif
__device__ __forceinline__ void g53_ld_str(g53_u4 (&c)[8], const uint8_t *p, int stride)
{
    g53_gv4 *q = (g53_gv4 *)p;
    const int st = stride >> 4;
#pragma unroll
    for (int k = 0; k < 8; k++) c[k] = q[k * st];
}

/* The chunk trade of a coalesced G or D item through the wave's 8 KB of LDS. Chunk n (16
 * bytes) of the item is chunk n % 8 of block n / 8 in the lane order of the block-per-lane
 * layout (a G item: blocks 0-31 the gate row, 32-63 the up row; a D item: 16 blocks per row,
 * four rows), stored at chunk position n ^ ((n >> 3) & 15): every 16 lanes of a store (16
 * consecutive n) and of a load (chunk q of 16 consecutive blocks) then cover all 64 banks. */
__device__ __forceinline__ void g53_xpose(g53_u4 (&c)[8], g53_u4 *xw, bool gitem, int lane)
{
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int n = gitem ? ((lane >> 5) * 256 + k * 32 + (lane & 31)) : (k * 64 + lane);
        xw[n ^ ((n >> 3) & 15)] = c[k];
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int q = 0; q < 8; q++) c[q] = xw[(8 * lane + q) ^ (lane & 15)];
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
}

__global__ void __launch_bounds__(G53_DEC_NT, 1) k_dec_layer(G53LayerArgs a)
{
    __shared__ __attribute__((aligned(16))) float xs[G53_DEC_NBE * G53_PADB];        /* padded x   */
    __shared__ __attribute__((aligned(16))) float actl[G53_DEC_NENT][G53_DEC_NBI * G53_PADB];
    __shared__ __attribute__((aligned(16))) double pw[G53_DEC_NT / 64][64];           /* row terms  */
    __shared__ g53_u4 xpw[G53_DEC_NT / 64][512];                                      /* chunk trade */
    __shared__ G53hExpert st[G53_DEC_MAXK + 1];
    __shared__ float biasl[G53_DEC_MAXNE];
    __shared__ float sw[64];
    __shared__ int sidx[16], ebuf[64];
    __shared__ uint32_t kbuf[64];
    __shared__ uint64_t etab[32];                      /* the exponential's table */
    __shared__ float cvals[G53_DEC_MAXRG][G53_DEC_RPD][G53_DEC_MAXK + 1];
    /* ent_ver[e]: activation halves copied into entry e so far; ent_used[e]: D items done with
     * it; routed: the routing and the routed slots' descriptors are in st[] and sw[] */
    __shared__ int qctr, ndone, routed, dready, ent_ver[G53_DEC_NENT], ent_used[G53_DEC_NENT];
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = a.K, hs = a.shared ? 1 : 0, nslots = K + hs;
    const int G = gridDim.x, b = blockIdx.x;

    G53List l;
    l.K = K;
    l.hs = hs;
    l.nR = a.NE > b ? (a.NE - 1 - b) / G + 1 : 0;
    l.g_lo = (int)((long)G53_DEC_I * b / G);
    l.g_n = (int)((long)G53_DEC_I * (b + 1) / G) - l.g_lo;
    l.rg_lo = (int)((long)G53_DEC_NGRP * b / G);
    l.n_rg = (int)((long)G53_DEC_NGRP * (b + 1) / G) - l.rg_lo;
    l.i_s = 0;
    l.i_sd = l.i_s + hs * l.g_n;
    l.i_g = l.i_sd + K * l.g_n;
    l.n = l.i_g + nslots * (2 + l.n_rg);
    const int ndone_all = nslots * l.n_rg;

    G53_TRACE(0);
    /* the router rows go out first: waves 0 .. nR-1 take rows b, b + G, ... */
    g53_u4 cr[8];
    if (w < l.nR) g53_ld_str(cr, (const uint8_t *)(a.router + (size_t)(b + w * G) * G53_DEC_E + lane * 64), 16);
    const int words = (int)(sizeof(G53hExpert) / 4);
    /* the descriptor table staged in the waiting waves' chunk-trade LDS, when it fits */
    uint2 *dtab = (uint2 *)xpw[G53_DEC_EARLY];
    const bool dstage = a.NE * (int)sizeof(G53hExpert) <= G53_DEC_DTAB;
    if (threadIdx.x < words) ((int *)&st[K])[threadIdx.x] = hs ? ((const int *)a.shared)[threadIdx.x] : 0;
    for (int e = threadIdx.x; e < a.NE; e += G53_DEC_NT) biasl[e] = a.bias[e];
    if (threadIdx.x == 0) { qctr = 0; ndone = 0; routed = 0; dready = 0; }
    if (threadIdx.x < 32) etab[threadIdx.x] = g53_exp2_tab_dev[threadIdx.x];
    if (threadIdx.x < G53_DEC_NENT) { ent_ver[threadIdx.x] = 0; ent_used[threadIdx.x] = 0; }
    for (int q = threadIdx.x; q < G53_DEC_E / 4; q += G53_DEC_NT) {
        const float4 v = ((const float4 *)a.x)[q];
        *(float4 *)(xs + (q >> 5) * G53_PADB + 4 * (q & 31)) = v;
    }
    if (w < l.nR) {
        /* the score of router row b + w G, published before the barrier: x is read straight
         * from memory, so the routing does not wait for the other waves' staging */
        const double d = g53_router_row(cr, a.x, lane);
        if (lane == 0) g53_st_tag(a.score + b + w * G, g53_tag(a.epoch, g53_sigmoidf_tab((float)d, g53_exp2_tab_dev)));
    }
    __syncthreads();
    if (threadIdx.x == 0 && hs && st[K].gate.w && !g53_desc_ok(st[K])) {
        st[K].gate.w = nullptr;                        /* unusable: flagged, contributes zero */
        if (b == 0) g53_flag_err(a.err, 8);
    }
    __syncthreads();
    G53_TRACE(8);

    g53_u64 tw_act = 0, tw_comp = 0, n_items = 0, n_stale = 0, n_stale2 = 0, tw_sh = 0, tw_use = 0, tw_d = 0, tw_mem = 0;
    auto claim = [&]() -> int {
        int i = 0;
        if (lane == 0) i = g53_lds_add(&qctr, 1);
        return __builtin_amdgcn_readfirstlane(i);
    };

    /* the routing item: top-k, weights, the chosen experts' descriptors (reference
     * src/core/glm53f_ops.c:945-976) */
    auto route = [&]() {
        G53_TRACE(11);
        bool ok;
        g53_u64 t_seen = 0, t_tau = 0, t_rank = 0;
        int n_polls = 0;
        if (a.NE <= 64 * 5)
            ok = g53_route_wave<5>(a.score, biasl, a.NE, K, a.norm_topk, a.routed_scale, a.epoch, sidx, sw, kbuf, ebuf,
                                   a.err, lane, t_seen, n_polls, t_tau, t_rank, a.spin);
        else
            ok = g53_route_wave<G53_DEC_MAXNE / 64>(a.score, biasl, a.NE, K, a.norm_topk, a.routed_scale, a.epoch, sidx,
                                                    sw, kbuf, ebuf, a.err, lane, t_seen, n_polls, t_tau, t_rank, a.spin);
        if (a.trace && lane == 0) { a.trace[(size_t)blockIdx.x * 32 + 15] = t_seen; a.trace[(size_t)blockIdx.x * 32 + 7] = n_polls; a.trace[(size_t)blockIdx.x * 32 + 1] = t_tau; a.trace[(size_t)blockIdx.x * 32 + 9] = t_rank; }
        if (!ok) {                                     /* scores missing: no routed slots */
            if (lane == 0) g53_flag_err(a.err, 1);
            if (lane < K) { sidx[lane] = -1; sw[lane] = 0.0f; }
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();
        }
        G53_TRACE(13);
        if (dstage) {                                  /* staged by the waiting waves */
            if (!g53_wait_lds(&dready, G53_DEC_NT / 64 - 1 - G53_DEC_EARLY) && lane == 0) g53_flag_err(a.err, 1);
            for (int q = lane; q < K * words; q += 64) {
                const int j = q / words, ex = sidx[j];
                ((int *)st)[q] = (ex >= 0 && ex < a.NE) ? ((const int *)dtab)[ex * words + q % words] : 0;
            }
        } else {                                       /* every load in flight at once */
            constexpr int NQ = (G53_DEC_MAXK * (int)(sizeof(G53hExpert) / 4) + 63) / 64;
            int dv[NQ];
#pragma unroll
            for (int i = 0; i < NQ; i++) {
                const int q = lane + 64 * i, j = min(q / words, K - 1), ex = sidx[j];
                dv[i] = (q < K * words && ex >= 0 && ex < a.NE) ? ((const int *)&a.experts[ex])[q % words] : 0;
            }
#pragma unroll
            for (int i = 0; i < NQ; i++)
                if (lane + 64 * i < K * words) ((int *)st)[lane + 64 * i] = dv[i];
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        if (lane < K && st[lane].gate.w && !g53_desc_ok(st[lane])) {
            st[lane].gate.w = nullptr;                 /* unusable: flagged, contributes zero */
            g53_flag_err(a.err, 8);
        }
        if (b == 0 && lane < K) {
            if (a.idx_out) a.idx_out[lane] = sidx[lane];
            if (a.w_out) a.w_out[lane] = sw[lane];
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        G53_CBAR();
        if (lane == 0) g53_lds_add(&routed, 1);
        G53_TRACE(14);
    };

    /* multiply one item whose codes are in c[] */
    auto compute = [&](const G53Item &it, const g53_u4 (&c)[8], float sc, bool loaded) {
        if (it.kind == G53_IT_G) {
            if (!loaded) return;                             /* expert not there */
            const float v = g53_gateup_pair(c, sc, xs, pw[w], a.limit, etab, lane);
            if (lane == 0) g53_st_tag(a.act + (size_t)it.s * G53_DEC_I + it.r, g53_tag(a.epoch, v));
            return;
        }
        const int e = it.t % G53_DEC_NENT;
        if (it.kind == G53_IT_A) {
            /* half of slot s's activations: check the epochs (re-reading stale values) and
             * store the values into entry t % NENT once its previous slot is done with it */
            const int use = it.t / G53_DEC_NENT;
            /* the entry's previous slot must be done with it, also when this slot is absent:
             * its count of copied halves must not run ahead of the previous slot's copies */
            if (use > 0 && g53_lds_ld(&ent_used[e]) < use * l.n_rg) {
                const g53_u64 t0 = __builtin_amdgcn_s_memrealtime();
                if (!g53_wait_lds(&ent_used[e], use * l.n_rg) && lane == 0) g53_flag_err(a.err, 1);
                tw_use += __builtin_amdgcn_s_memrealtime() - t0;
            }
            if (!st[it.s].gate.w) {                          /* not used by any D item */
                G53_CBAR();
                if (lane == 0) g53_lds_add(&ent_ver[e], 1);
                return;
            }
            /* value 2k of this lane: c[k].x (value) / c[k].y (epoch); value 2k+1: c[k].z / c[k].w */
            uint32_t pending = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                if (c[k].y != a.epoch) pending |= 1u << (2 * k);
                if (c[k].w != a.epoch) pending |= 1u << (2 * k + 1);
            }
            const int i0 = it.r * 1024 + lane * 16;          /* 16 values within one block */
            float *dst = actl[e] + (i0 >> 7) * G53_PADB + (i0 & 127);
#pragma unroll
            for (int k = 0; k < 4; k++)
                *(float4 *)(dst + 4 * k) = make_float4(__uint_as_float(c[2 * k].x), __uint_as_float(c[2 * k].z),
                                                       __uint_as_float(c[2 * k + 1].x), __uint_as_float(c[2 * k + 1].z));
            if (__ballot(pending != 0)) {
                /* stale values (read from a line this XCD's L2 took before they were written):
                 * re-read them coherently until their epochs are current, and store each back
                 * with a plain store, which refreshes the stale line for the workgroups of this
                 * XCD that read it later (the value stored is the one already in memory) */
                const g53_u64 t0 = __builtin_amdgcn_s_memrealtime();
                n_stale += __popc(pending);
                g53_u64 *src = a.act + (size_t)it.s * G53_DEC_I + it.r * 1024 + lane * 16;
                const __amdgpu_buffer_rsrc_t rsrc = g53_rsrc(a.act + (size_t)it.s * G53_DEC_I + it.r * 1024);
                int spins = 0;
                while (__ballot(pending != 0)) {
                    if (++spins > a.spin) { if (lane == 0) g53_flag_err(a.err, 1); break; }
#pragma unroll
                    for (int h = 0; h < 16; h += 4) {
                        g53_u64 t[4];
#pragma unroll
                        for (int k = 0; k < 4; k++)
                            t[k] = (pending & (1u << (h + k))) ? g53_ld_coh64(rsrc, 8 * (lane * 16 + h + k)) : 0ull;
#pragma unroll
                        for (int k = 0; k < 4; k++)
                            if ((pending & (1u << (h + k))) && (unsigned)(t[k] >> 32) == a.epoch) {
                                dst[h + k] = __uint_as_float((uint32_t)t[k]);
                                src[h + k] = t[k];
                                pending &= ~(1u << (h + k));
                            }
                    }
                    if (spins == 1) n_stale2 += __popc(pending);
                    if (__ballot(pending != 0)) g53_backoff();
                }
                if (it.s == K) tw_sh += __builtin_amdgcn_s_memrealtime() - t0;
                else tw_act += __builtin_amdgcn_s_memrealtime() - t0;
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();
            G53_CBAR();
            if (lane == 0) g53_lds_add(&ent_ver[e], 1);
            return;
        }
        /* D item */
        float v = 0.0f;
        if (loaded) {
            const int want = 2 * (it.t / G53_DEC_NENT + 1);
            if (g53_lds_ld(&ent_ver[e]) < want) {
                const g53_u64 t0 = __builtin_amdgcn_s_memrealtime();
                if (!g53_wait_lds(&ent_ver[e], want) && lane == 0) g53_flag_err(a.err, 1);
                tw_d += __builtin_amdgcn_s_memrealtime() - t0;
            }
            const int bb = lane & 15;
            v = (float)g53_row_sum<16>(g53_blk_pad(c, actl[e] + bb * G53_PADB) * (double)sc, pw[w], lane);
        }
        if ((lane & 15) == 0) cvals[it.r - l.rg_lo][lane >> 4][it.s] = v;
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        G53_CBAR();
        int fin = 0;
        if (lane == 0) {
            g53_lds_add(&ent_used[e], 1);
            fin = g53_lds_add(&ndone, 1) == ndone_all - 1;
        }
        if (__builtin_amdgcn_readfirstlane(fin)) {
            /* every contribution of the workgroup's rows is in: combine them (reference
             * src/core/glm53f_ops.c:1329-1340) */
            G53_CBAR();
            const int m = lane >> 2, r = lane & 3;
            if (m < l.n_rg) {
                double acc = 0.0;
                for (int j = 0; j < K; j++) acc = acc + (double)sw[j] * (double)cvals[m][r][j];
                float o = (float)acc;
                if (hs) o = o + cvals[m][r][K];
                a.out[(l.rg_lo + m) * G53_DEC_RPD + r] = o;
            }
        }
    };

    /* ---- the item loop ----
     * Two code buffers alternate: each half-pass claims an item and issues its loads into the
     * free buffer (from one place, so the compiler keeps them in flight), then multiplies the
     * item in the other buffer. While a wave waits for one item's codes, the next item's are
     * already on their way. An item of a routed slot waits for the routing before its loads
     * are issued. */
    auto next_item = [&]() -> G53Item {
        const int i = claim();
        G53Item it = i < l.n ? g53_item(l, i, b, G) : G53Item{G53_IT_NONE, 0, 0, 0};
        /* uniform by construction; said so, so that the loop's branches stay scalar */
        it.kind = __builtin_amdgcn_readfirstlane(it.kind);
        it.s = __builtin_amdgcn_readfirstlane(it.s);
        it.r = __builtin_amdgcn_readfirstlane(it.r);
        it.t = __builtin_amdgcn_readfirstlane(it.t);
        return it;
    };
    auto issue = [&](const G53Item &nt, g53_u4 (&c)[8], float &scv) -> bool {
        if ((nt.kind == G53_IT_G || nt.kind == G53_IT_A || nt.kind == G53_IT_D) && nt.s < K &&
            g53_lds_ld(&routed) == 0) {
            if (!g53_wait_lds(&routed, 1) && lane == 0) g53_flag_err(a.err, 1);
        }
        const uint8_t *p;
        const float *ps;
        int stride;
        const bool r = g53_addr(nt, st, a.act, a.router, a.x, lane, p, ps, stride);
        g53_ld_str(c, p, stride);
        scv = *(const g53_gf *)ps;
        return __builtin_amdgcn_readfirstlane((int)r) != 0;   /* uniform: no exec-masked paths */
    };
    auto run = [&](const G53Item &it, g53_u4 (&c)[8], float scv, bool loaded) {
        const g53_u64 tw0 = __builtin_amdgcn_s_memrealtime();
        g53_touch(c, scv);
        if (it.kind == G53_IT_NONE) return;
        const g53_u64 tc0 = __builtin_amdgcn_s_memrealtime();
        tw_mem += tc0 - tw0;
        if (loaded && (it.kind == G53_IT_G || it.kind == G53_IT_D)) g53_xpose(c, xpw[w], it.kind == G53_IT_G, lane);
        compute(it, c, scv, loaded);
        tw_comp += __builtin_amdgcn_s_memrealtime() - tc0;
        n_items++;
    };
    if (w == G53_DEC_NT / 64 - 1) route();
    /* only a few waves stream before the routing is known, so that the loads, the
     * publications and the coherent reads of the routing are not queued behind a saturated
     * memory system */
    if (w >= G53_DEC_EARLY && w < G53_DEC_NT / 64 - 1) {
        /* waves that wait for the routing first copy the expert descriptor table into their
         * (still unused) chunk-trade LDS, so that the routing wave picks the chosen ones from
         * there; for a table too large for it they only touch it into this XCD's L2 */
        constexpr int NP = G53_DEC_NT / 64 - 1 - G53_DEC_EARLY;
        constexpr int PER = (G53_DEC_DTAB / 8 + NP * 64 - 1) / (NP * 64);
        const int n8 = a.NE * (int)(sizeof(G53hExpert) / 8);
        const uint2 *t8 = (const uint2 *)a.experts;
        const int base = (w - G53_DEC_EARLY) * 64 + lane;
        if (dstage) {
            uint2 v[PER];
#pragma unroll
            for (int k = 0; k < PER; k++) v[k] = base + k * NP * 64 < n8 ? t8[base + k * NP * 64] : make_uint2(0u, 0u);
#pragma unroll
            for (int k = 0; k < PER; k++)
                if (base + k * NP * 64 < n8) dtab[base + k * NP * 64] = v[k];
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();
            G53_CBAR();
            if (lane == 0) g53_lds_add(&dready, 1);
        } else {
            for (int q = base; q < n8; q += 4 * NP * 64) {
                uint2 v0 = t8[q], v1 = q + NP * 64 < n8 ? t8[q + NP * 64] : v0;
                uint2 v2 = q + 2 * NP * 64 < n8 ? t8[q + 2 * NP * 64] : v0;
                uint2 v3 = q + 3 * NP * 64 < n8 ? t8[q + 3 * NP * 64] : v0;
                asm volatile("" ::"v"(v0.x), "v"(v1.x), "v"(v2.x), "v"(v3.x));
            }
        }
    }
    if (w >= G53_DEC_EARLY && g53_lds_ld(&routed) == 0) {
        if (!g53_wait_lds(&routed, 1) && lane == 0) g53_flag_err(a.err, 1);
    }
    g53_u4 ca[8], cb[8];
    float sa = 0.0f, sb = 0.0f;
    G53Item ia = next_item();
    bool la = issue(ia, ca, sa);
    G53Item ib = next_item();
    bool lb = issue(ib, cb, sb);
    /* One exit, at the top, and no branch around either half: the items are claimed in order,
     * so once one is none every later one is, and a none item only waits for its (dummy)
     * loads. Every path through the body then leaves buffer a's loads older than buffer b's,
     * so the compiler waits for exactly one buffer at a time. */
    while (ia.kind != G53_IT_NONE) {
        run(ia, ca, sa, la);
        ia = next_item();
        la = issue(ia, ca, sa);
        run(ib, cb, sb, lb);
        ib = next_item();
        lb = issue(ib, cb, sb);
    }
    if (w < 4) G53_TRACE(2 + w);
    if (a.trace && lane == 0 && w < 4) {
        g53_u64 *tr = a.trace + (size_t)blockIdx.x * 32;
        tr[16 + w] = tw_sh + tw_act; tr[20 + w] = tw_use; tr[6] = n_stale2; tr[24 + w] = tw_d; tr[28 + w] = tw_mem; (void)n_stale; (void)tw_comp; (void)n_items;
    }
}

/* ------------------------------------------------------------------ host side ---- */
static int g_dec_grid1 = -1;             /* workgroups of k_dec_layer, 0 = unavailable     */
static unsigned g_dec_epoch = 0;         /* epoch of the last launch                        */
static void *g_dec_buf = nullptr;        /* tagged scores | tagged activations              */
static size_t g_dec_buf_bytes = 0;
static int g_dec_enabled = 1;
static g53_u64 *g_dec_trace = nullptr;

static int g53_dec_shape(const G53hMoeLayer *L)
{
    if (L->block_c != 128 || L->hidden != G53_DEC_E || L->inter != G53_DEC_I || L->router_dt != 1) return 0;
    if (L->topk < 1 || L->topk > G53_DEC_MAXK || L->n_experts > G53_DEC_MAXNE) return 0;
    return 1;
}

extern "C" int g53h_set_decode_trace(void *dev_buf)
{
    g_dec_trace = (g53_u64 *)dev_buf;
    return 0;
}

extern "C" int g53h_set_fused_decode(int on)
{
    const int old = g_dec_enabled;
    g_dec_enabled = on != 0;
    return old;
}

int g53h_decode_fused(float *out, const float *x, const G53hMoeLayer *L, int *idx_out, float *w_out)
{
    if (!g_dec_enabled || !g53_dec_shape(L)) return 1;     /* not handled: caller falls back */
    const int K = L->topk, NE = L->n_experts;
    const int cus = g53h_num_cus();
    if (g_dec_grid1 < 0) {
        int per = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, (const void *)k_dec_layer, G53_DEC_NT, 0) != hipSuccess ||
            per < 1) {
            (void)hipGetLastError();
            g_dec_grid1 = 0;
        } else {
            g_dec_grid1 = cus;
            /* every workgroup owns at most G53_DEC_MAXRG row groups */
            if ((G53_DEC_NGRP + g_dec_grid1 - 1) / g_dec_grid1 > G53_DEC_MAXRG) g_dec_grid1 = 0;
        }
    }
    if (!g_dec_grid1) return 1;
    /* tagged scores [MAXNE] | tagged act [ROT][MAXK + 1][I], allocated and cleared once, so
     * that no tagged word carries a live epoch. The tagged activations rotate over ROT copies
     * by epoch, so a copy is reused only ROT launches later. */
    const size_t off_act = (size_t)G53_DEC_MAXNE * 8;
    const size_t act_copy = (size_t)(G53_DEC_MAXK + 1) * G53_DEC_I * 8;
    const size_t bytes = off_act + G53_DEC_ROT * act_copy;
    if (!g_dec_buf) {
        G53_TRY(hipMalloc(&g_dec_buf, bytes));
        G53_TRY(hipMemset(g_dec_buf, 0, bytes));
        G53_TRY(hipDeviceSynchronize());
        g_dec_buf_bytes = bytes;
        g_dec_epoch = 0;
    }
    if (++g_dec_epoch == 0) {                              /* wrapped: clear and start over */
        G53_TRY(hipStreamSynchronize(g53h_stream()));
        G53_TRY(hipMemset(g_dec_buf, 0, g_dec_buf_bytes));
        G53_TRY(hipDeviceSynchronize());
        g_dec_epoch = 1;
    }
    char *buf = (char *)g_dec_buf;
    G53LayerArgs e;
    e.out = out; e.x = x; e.router = (const uint16_t *)L->router; e.bias = L->bias;
    e.experts = L->experts; e.shared = L->shared;
    e.score = (g53_u64 *)buf;
    e.act = (g53_u64 *)(buf + off_act + (g_dec_epoch % G53_DEC_ROT) * act_copy);
    e.err = g53h_errblock(); e.idx_out = idx_out; e.w_out = w_out;
    e.NE = NE; e.K = K; e.norm_topk = L->norm_topk; e.epoch = g_dec_epoch;
    e.spin = g53h_spin_limit(); e.routed_scale = L->routed_scale; e.limit = L->swiglu_limit; e.trace = g_dec_trace;
    g53h_prof_mark(G53_PROF_START);
    hipLaunchKernelGGL(k_dec_layer, dim3(g_dec_grid1), dim3(G53_DEC_NT), 0, g53h_stream(), e);
    G53_LAUNCHED("k_dec_layer");
    g53h_prof_mark(G53_PROF_FUSED);
    return 0;
}

extern "C" int g53h_decode_errors(void)
{
    if (g53h_ready()) return 0;
    int e[2] = {0, 0};
    if (hipStreamSynchronize(g53h_stream()) != hipSuccess) return -1;
    if (hipMemcpy(e, g53h_errblock(), sizeof e, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    if ((e[0] | e[1]) && hipMemset(g53h_errblock(), 0, sizeof e) != hipSuccess) return -1;
    return e[0] | e[1];
}

extern "C" int g53h_decode_grid(void) { return g_dec_grid1; }
