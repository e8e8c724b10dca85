/* g53h_decode.hip - single-token decode of one MoE layer in one persistent launch.
 *
 * The layer (reference src/core/glm53f_ops.c:1144-1342 at T = 1) is three phases over one
 * grid of co-resident workgroups, separated by two grid barriers:
 *
 *   A  router dot products (one wave per expert) and, on the remaining waves, the shared
 *      expert's gate and up rows, which do not depend on the routing;
 *   B  every workgroup reads the scores and selects the top-k itself (a few microseconds of
 *      redundant work instead of another barrier), then the routed experts' gate and up rows;
 *   C  down rows of every slot; the last of a row group's slots to finish combines the row
 *      group in double in top-k order and adds the shared expert.
 *
 * Arithmetic is the reference's, bit for bit (see g53h_gemv.h). Values handed from one
 * workgroup to another (scores, activations, contributions, counters) use agent-scope
 * relaxed accesses, which are coherent across the XCDs' L2 caches; each handoff is ordered by
 * waiting for the stores to complete before the counter that publishes them is advanced.
 *
 * Co-residency: the grid is sized from the occupancy the runtime reports, and every wait on
 * another workgroup is bounded; a wait that runs out sets an error flag (read by
 * g53h_decode_errors) and the workgroup leaves, so the grid always drains.
 */
#include <hip/hip_runtime.h>
#include <math.h>

#include "g53h.h"
#include "g53h_core.h"
#include "g53h_gemv.h"
#include "g53h_kern.h"
#include "g53h_runtime.h"

#define G53_DEC_MAXK 16            /* top-k handled by the fused kernel            */
#define G53_DEC_MAXNE 1024
#define G53_SPIN_LIMIT (1 << 22)   /* sleep-polls before a grid wait gives up      */

struct G53DecodeArgs {
    float *out;
    const float *x;
    const void *router;
    const float *bias;
    const G53hExpert *experts;
    const G53hExpert *shared;
    float *score, *choice;         /* [NE]                                          */
    float *act;                    /* [nslots][I]                                   */
    float *contrib;                /* [nslots][E]                                   */
    int *grp_cnt;                  /* [E / RPW_D], zero between launches            */
    int *bar;                      /* grid barrier counter, monotonic               */
    int *err;                      /* set to 1 when a wait gives up                 */
    int *idx_out;
    float *w_out;
    int router_dt, E, I, NE, K, norm_topk, nslots;
    int bar_base;
    float routed_scale, limit;
    int pb_rows;                   /* rows of the per-wave term buffer              */
    unsigned long long *trace;     /* optional: [grid][8] phase timestamps          */
};

/* Phase timestamps (100 MHz real-time counter) for the trace buffer, thread 0 only. */
#define G53_TRACE(k) do { if (a.trace && threadIdx.x == 0) \
    a.trace[(size_t)blockIdx.x * 8 + (k)] = __builtin_amdgcn_s_memrealtime(); } while (0)

/* Grid barrier: returns false (and sets *err) if the other workgroups did not arrive. */
__device__ bool g53_grid_sync(int *bar, int target, int *err)
{
    __builtin_amdgcn_s_waitcnt(0);                  /* this thread's stores are complete */
    __syncthreads();
    __shared__ int ok;
    if (threadIdx.x == 0) {
        __hip_atomic_fetch_add(bar, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int spins = 0;
        ok = 1;
        while ((int)((unsigned)g53_ld_agent_i(bar) - (unsigned)target) < 0) {
            if (++spins > G53_SPIN_LIMIT) {
                ok = 0;
                __hip_atomic_fetch_or(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(8);
        }
    }
    __syncthreads();
    return ok != 0;
}

/* One chunk of gate/up rows: OPS values of o of expert m (lanes: gate o, up o, gate o+1, ...).
 * Writes the lane's block term to pw[row][b]. */
template <int NBE>
__device__ __forceinline__ void g53_gu_issue(uint4 (&c)[8], float &sc, const G53hExpert &ex, int o, int E, int up,
                                             int b)
{
    const G53hMat &m = up ? ex.up : ex.gate;
    g53_ld_blk(c, m.w + (size_t)o * E + b * 128);
    sc = ((g53_gf *)m.s)[(size_t)(o / m.br) * m.scols + b];
}

/* Gate/up rows of a list of chunks (chunk c -> slot c / cps of the table, o = (c % cps)*OPS +
 * ol), taken in grid-stride order starting at c0 with stride nw; then each buffered row is
 * summed in block order and the SwiGLU of each (gate, up) pair goes to act[slot][o]. */
template <int NBE>
__device__ void g53_gateup_chunks(const G53hExpert *st, int nchunks, int c0, int nw, const float *xs, double *pw,
                                  float *act, int I, int E, float limit)
{
    constexpr int RPW = 64 / NBE, OPS = RPW / 2, PST = NBE + 1;
    const int lane = threadIdx.x & 63;
    const int b = lane % NBE, rw = lane / NBE, ol = rw >> 1, up = rw & 1;
    const int cps = I / OPS;
    const float *xb = xs + b * 128;
    int steps = 0;
    for (int c = c0; c < nchunks; c += nw) steps++;
    if (steps == 0) return;
    uint4 cur[8];
    float sc = 0.0f;
    int c = c0;
    bool have = st[c / cps].gate.w != nullptr;
    if (have) g53_gu_issue<NBE>(cur, sc, st[c / cps], (c % cps) * OPS + ol, E, up, b);
    for (int j = 0; j < steps; j++, c += nw) {
        const int cn = c + nw;
        const bool hn = j + 1 < steps && st[cn / cps].gate.w != nullptr;
        uint4 nxt[8];
        float scn = 0.0f;
        if (hn) g53_gu_issue<NBE>(nxt, scn, st[cn / cps], (cn % cps) * OPS + ol, E, up, b);
        if (have) pw[(j * RPW + rw) * PST + b] = g53_blk_lds(cur, xb, b) * (double)sc;
        have = hn;
        sc = scn;
#pragma unroll
        for (int k = 0; k < 8; k++) cur[k] = nxt[k];
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    const int jr = lane / RPW, rr = lane % RPW, cr = c0 + jr * nw;
    const bool mine = lane < steps * RPW && st[cr / cps].gate.w != nullptr;
    float v = 0.0f;
    if (mine) {
        double acc = 0.0;
        const double *pr = pw + lane * PST;
        for (int bb = 0; bb < NBE; bb++) acc = acc + pr[bb];
        v = (float)acc;
    }
    const float u = __shfl_down(v, 1);
    if (mine && !(rr & 1)) {
        const int s = cr / cps, o = (cr % cps) * OPS + (rr >> 1);
        g53_st_agent(act + (size_t)s * I + o, g53_swiglu1(v, u, limit));
    }
    __builtin_amdgcn_wave_barrier();
}

template <int NBE, int NBI>
__global__ void __launch_bounds__(256, 2) k_moe_decode(G53DecodeArgs a)
{
    constexpr int RPD = 64 / NBI, PSD = NBI + 1;
    __shared__ __attribute__((aligned(16))) float xs[NBE * 128];
    __shared__ G53hExpert st[G53_DEC_MAXK + 1];
    __shared__ int sel[G53_DEC_MAXK];
    __shared__ float sw[G53_DEC_MAXK];
    __shared__ uint32_t kbuf[G53_DEC_MAXK];
    __shared__ int ebuf[G53_DEC_MAXK];
    /* phase B keeps the scores here, phase C the four waves' activations */
    __shared__ __attribute__((aligned(16))) float uni[4 * NBI * 128 > 2 * G53_DEC_MAXNE ? 4 * NBI * 128
                                                                                     : 2 * G53_DEC_MAXNE];
    float *ch = uni, *scs = uni + G53_DEC_MAXNE;
    extern __shared__ double pbd[];                 /* [4][pb_rows * max(PST)]           */
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nw = gridDim.x * 4, wave = blockIdx.x * 4 + w;
    const int E = a.E, I = a.I, NE = a.NE, K = a.K, nslots = a.nslots;
    double *pw = pbd + (size_t)w * a.pb_rows * (NBE + 1);

    /* ---- phase A: router dot products; the shared expert's gate/up ---- */
    G53_TRACE(0);
    g53_vec_to_lds(xs, a.x, E, threadIdx.x, 256);
    if (threadIdx.x < (int)(sizeof(G53hExpert) / 4) && a.shared)
        ((int *)&st[K])[threadIdx.x] = ((const int *)a.shared)[threadIdx.x];
    __syncthreads();
    for (int e = wave; e < NE; e += nw) {
        const float d = g53_router_dot(a.router, a.router_dt, e, E, a.x, lane);
        if (lane == 0) {
            const float s = g53_sigmoidf(d);
            g53_st_agent(a.score + e, s);
            g53_st_agent(a.choice + e, s + a.bias[e]);
        }
    }
    if (a.shared) {
        constexpr int OPS = 32 / NBE;
        const int nch = I / OPS;
        int c0 = (wave - NE) % nw;
        if (c0 < 0) c0 += nw;
        g53_gateup_chunks<NBE>(st + K, nch, c0, nw, xs, pw, a.act + (size_t)K * I, I, E, a.limit);
    }
    G53_TRACE(1);
    if (!g53_grid_sync(a.bar, a.bar_base + gridDim.x, a.err)) return;
    G53_TRACE(2);

    /* ---- phase B: routing (every workgroup), routed gate/up ---- */
    {
        const int NE4 = (NE + 3) & ~3;
        for (int q = threadIdx.x; q < NE4 / 4; q += 256) {
            const float4 cv = g53_ld4_agent(a.choice, 16 * q), sv = g53_ld4_agent(a.score, 16 * q);
            *(float4 *)(ch + 4 * q) = cv;
            *(float4 *)(scs + 4 * q) = sv;
        }
    }
    __syncthreads();
    if (w == 0) g53_topk_wave(ch, NE, K, sel, kbuf, ebuf);
    __syncthreads();
    if (threadIdx.x == 0) {
        int bad = 0;
        for (int j = 0; j < K; j++) {
            if (sel[j] < 0) { bad = 1; sel[j] = 0; }
            sw[j] = scs[sel[j]];
        }
        if (bad) __hip_atomic_fetch_or(a.err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (a.norm_topk) {
            double s = 0.0;
            for (int j = 0; j < K; j++) s += (double)sw[j];
            for (int j = 0; j < K; j++) sw[j] = (float)((double)sw[j] / (s + 1e-20));
        }
        for (int j = 0; j < K; j++) sw[j] = sw[j] * a.routed_scale;
        if (blockIdx.x == 0) {
            for (int j = 0; j < K; j++) {
                if (a.idx_out) a.idx_out[j] = sel[j];
                if (a.w_out) a.w_out[j] = sw[j];
            }
        }
    }
    __syncthreads();
    {
        const int words = (int)(sizeof(G53hExpert) / 4);
        for (int q = threadIdx.x; q < K * words; q += 256)
            ((int *)&st[q / words])[q % words] = ((const int *)&a.experts[sel[q / words]])[q % words];
    }
    __syncthreads();
    G53_TRACE(3);
    {
        constexpr int OPS = 32 / NBE;
        g53_gateup_chunks<NBE>(st, K * (I / OPS), wave, nw, xs, pw, a.act, I, E, a.limit);
    }

    /* prefetch this wave's first down chunk before waiting */
    const int nwc = (nw / nslots) * nslots, gstride = nw / nslots, ngrp = E / RPD;
    const int s_c = wave % nslots, b_c = lane % NBI, rw_c = lane / NBI;
    const G53hExpert &exc = st[s_c];
    const bool cwave = wave < nwc && exc.gate.w != nullptr;
    uint4 cur[8];
    float sc = 0.0f;
    int g = wave / nslots;
    if (cwave && g < ngrp) {
        const int d = g * RPD + rw_c;
        g53_ld_blk(cur, exc.down.w + (size_t)d * I + b_c * 128);
        sc = ((g53_gf *)exc.down.s)[(size_t)(d / exc.down.br) * exc.down.scols + b_c];
    }
    G53_TRACE(4);
    if (!g53_grid_sync(a.bar, a.bar_base + 2 * gridDim.x, a.err)) return;
    G53_TRACE(5);

    /* ---- phase C: down rows of slot s_c, row groups g, g + gstride, ...; combine ---- */
    if (wave >= nwc) return;
    float *av = uni + (size_t)w * NBI * 128;          /* the scores are no longer read */
    for (int c4 = lane; c4 < I / 4; c4 += 64) {          /* this slot's activation, swizzled */
        const int i = 4 * c4, blk = i / 128, q = (i % 128) / 4;
        *(float4 *)(av + blk * 128 + 4 * (q ^ (blk & 31))) = g53_ld4_agent(a.act, ((int)s_c * I + i) * 4);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    if (w == 0) G53_TRACE(6);
    int steps = 0;
    for (int gg = g; gg < ngrp; gg += gstride) steps++;
    double *pc = pbd + (size_t)w * a.pb_rows * (NBE + 1);
    for (int j = 0; j < steps; j++) {
        const int gn = g + (j + 1) * gstride;
        const bool hn = cwave && j + 1 < steps;
        uint4 nxt[8];
        float scn = 0.0f;
        if (hn) {
            const int d = gn * RPD + rw_c;
            g53_ld_blk(nxt, exc.down.w + (size_t)d * I + b_c * 128);
            scn = ((g53_gf *)exc.down.s)[(size_t)(d / exc.down.br) * exc.down.scols + b_c];
        }
        if (cwave) pc[(j * RPD + rw_c) * PSD + b_c] = g53_blk_lds(cur, av + b_c * 128, b_c) * (double)sc;
        sc = scn;
#pragma unroll
        for (int k = 0; k < 8; k++) cur[k] = nxt[k];
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    /* lane r: row r % RPD of step r / RPD */
    const int jr = lane / RPD, rr = lane % RPD, gr = g + jr * gstride, dr = gr * RPD + rr;
    const bool mine = lane < steps * RPD;
    if (mine) {
        float v = 0.0f;
        if (cwave) {
            double acc = 0.0;
            const double *pr = pc + lane * PSD;
            for (int bb = 0; bb < NBI; bb++) acc = acc + pr[bb];
            v = (float)acc;
        }
        g53_st_agent(a.contrib + (size_t)s_c * E + dr, v);
    }
    __builtin_amdgcn_s_waitcnt(0);                        /* contributions complete */
    int last = 0;
    if (mine && rr == 0)
        last = __hip_atomic_fetch_add(a.grp_cnt + gr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nslots - 1;
    last = __shfl(last, lane - rr);
    if (mine && last) {
        double acc = 0.0;
        for (int j = 0; j < K; j++) acc = acc + (double)sw[j] * (double)g53_ld_agent(a.contrib + (size_t)j * E + dr);
        float o = (float)acc;
        if (nslots > K) o = o + g53_ld_agent(a.contrib + (size_t)K * E + dr);
        a.out[dr] = o;
        if (rr == 0) __hip_atomic_store(a.grp_cnt + gr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (w == 0) G53_TRACE(7);
}

/* ------------------------------------------------------------------ host side ---- */
static int g_dec_grid = -1;              /* workgroups of the fused kernel, 0 = unavailable */
static unsigned g_dec_epoch = 0;         /* barrier counter value at the next launch        */
static int *g_dec_state = nullptr;       /* [0] barrier counter, [1] error flags, [2..] group counters */

static int g53_dec_shape(const G53hMoeLayer *L)
{
    const int nslots = L->topk + (L->shared ? 1 : 0);
    if (L->block_c != 128 || L->hidden != 4096 || L->inter != 2048) return 0;
    if (L->topk > G53_DEC_MAXK || L->n_experts > G53_DEC_MAXNE || nslots < 1) return 0;
    return 1;
}

static int g_dec_enabled = 1;
static unsigned long long *g_dec_trace = nullptr;

extern "C" int g53h_set_decode_trace(void *dev_buf)
{
    g_dec_trace = (unsigned long long *)dev_buf;
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
    const int E = L->hidden, I = L->inter, K = L->topk, nslots = K + (L->shared ? 1 : 0);
    constexpr int NBE = 32, NBI = 16, RPD = 64 / NBI;
    const int cus = g53h_num_cus();
    /* term buffer rows: the most chunks one wave takes in any phase, times rows per chunk */
    auto rows_for = [&](int nwv) {
        const int a = (L->n_experts + I / 1 + nwv - 1) / nwv * 2;        /* phase A (upper bound) */
        const int bph = (K * I + nwv - 1) / nwv * 2;                       /* phase B               */
        const int c = ((E / RPD) + nwv / nslots - 1) / (nwv / nslots) * RPD;   /* phase C          */
        int r = a > bph ? a : bph;
        return r > c ? r : c;
    };
    if (g_dec_grid < 0) {
        int per = 0;
        const int rows = rows_for(8 * cus);
        const size_t dyn = (size_t)4 * rows * (NBE + 1) * sizeof(double);
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, (const void *)k_moe_decode<NBE, NBI>, 256, dyn) !=
                hipSuccess || per < 1) {
            (void)hipGetLastError();
            g_dec_grid = 0;
        } else {
            g_dec_grid = (per > 2 ? 2 : per) * cus;
        }
        if (g_dec_grid) {
            if (hipMalloc((void **)&g_dec_state, (2 + 4096) * sizeof(int)) != hipSuccess ||
                hipMemset(g_dec_state, 0, (2 + 4096) * sizeof(int)) != hipSuccess ||
                hipDeviceSynchronize() != hipSuccess) {
                (void)hipGetLastError();
                g_dec_grid = 0;
            }
        }
    }
    if (!g_dec_grid) return 1;
    const int nwv = 4 * g_dec_grid;
    const int rows = rows_for(nwv);
    if (rows > 64 || E / RPD > 4096) return 1;
    const size_t dyn = (size_t)4 * rows * (NBE + 1) * sizeof(double);
    char *ws = (char *)g53h_workspace((size_t)2 * L->n_experts * 4 + 256 + (size_t)nslots * (I + E) * 4 + 512);
    if (!ws) return -1;
    G53DecodeArgs a;
    a.out = out; a.x = x; a.router = L->router; a.bias = L->bias; a.experts = L->experts; a.shared = L->shared;
    a.score = (float *)ws;
    a.choice = a.score + L->n_experts;
    a.act = (float *)(ws + (((size_t)2 * L->n_experts * 4 + 255) & ~(size_t)255));
    a.contrib = a.act + (size_t)nslots * I;
    a.bar = g_dec_state;
    a.err = g_dec_state + 1;
    a.grp_cnt = g_dec_state + 2;
    a.idx_out = idx_out; a.w_out = w_out;
    a.router_dt = L->router_dt; a.E = E; a.I = I; a.NE = L->n_experts; a.K = K; a.norm_topk = L->norm_topk;
    a.nslots = nslots; a.bar_base = (int)g_dec_epoch;   /* wraps; compared as a difference */
    a.routed_scale = L->routed_scale; a.limit = L->swiglu_limit; a.pb_rows = rows; a.trace = g_dec_trace;
    g53h_prof_mark(G53_PROF_START);
    hipLaunchKernelGGL((k_moe_decode<NBE, NBI>), dim3(g_dec_grid), dim3(256), dyn, g53h_stream(), a);
    G53_LAUNCHED("k_moe_decode");
    g53h_prof_mark(G53_PROF_FUSED);
    g_dec_epoch += 2u * (unsigned)g_dec_grid;
    return 0;
}

extern "C" int g53h_decode_errors(void)
{
    if (g53h_ready() || !g_dec_state) return 0;
    int e = 0;
    if (hipStreamSynchronize(g53h_stream()) != hipSuccess) return -1;
    if (hipMemcpy(&e, g_dec_state + 1, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess) return -1;
    if (e) (void)hipMemset(g_dec_state + 1, 0, sizeof(int));
    return e;
}

extern "C" int g53h_decode_grid(void) { return g_dec_grid; }
