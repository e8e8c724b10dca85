/* g53h_runtime.hip - device selection, streams, memory, timing and the workspace. */
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "g53h.h"
#include "g53h_runtime.h"

static char        g_err[512];
static int         g_ready = 0;
static int         g_device = -1;
static int         g_cus = 0;
static hipStream_t g_stream = nullptr;
static hipStream_t g_copy = nullptr;
static hipEvent_t  g_ev[2] = {nullptr, nullptr};
static int         g_ev_next = 0;
static void       *g_ws = nullptr;
static size_t      g_ws_bytes = 0;
static int        *g_counters = nullptr;
static int        *g_errs = nullptr;   /* [0] k_dec_layer, [1] k_dec_tiled, [2] grouped path   */
static unsigned   *g_mbox = nullptr;   /* host mailbox: pinned, mapped, written by kernels      */
static unsigned   *g_mbox_d = nullptr; /* its device address                                    */
static uint8_t    *g_inbox = nullptr;  /* host inbox: pinned, mapped, read by kernels           */
static uint8_t    *g_inbox_d = nullptr;

extern "C" int g53h_fail(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return -1;
}

extern "C" int g53h_check(hipError_t e, const char *what, const char *file, int line)
{
    if (e == hipSuccess) return 0;
    return g53h_fail("%s failed at %s:%d: %s", what, file, line, hipGetErrorString(e));
}

extern "C" const char *g53h_error(void) { return g_err; }

extern "C" int g53h_device_count(void)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

extern "C" int g53h_init(int device)
{
    if (g_ready && device == g_device) return 0;
    if (g_ready) return g53h_fail("g53h_init: already bound to device %d", g_device);
    int n = 0;
    G53_TRY(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return g53h_fail("g53h_init: device %d of %d", device, n);
    G53_TRY(hipSetDevice(device));
    hipDeviceProp_t p;
    G53_TRY(hipGetDeviceProperties(&p, device));
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return g53h_fail("g53h_init: device %d is %s; this library is built for gfx950 only",
                         device, p.gcnArchName);
    g_cus = p.multiProcessorCount;
    /* default priority only: streams of other priorities are not used by this library */
    G53_TRY(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    G53_TRY(hipStreamCreateWithFlags(&g_copy, hipStreamNonBlocking));
    G53_TRY(hipEventCreate(&g_ev[0]));
    G53_TRY(hipEventCreate(&g_ev[1]));
    G53_TRY(hipMalloc((void **)&g_counters, 4096 * sizeof(int)));
    G53_TRY(hipMemset(g_counters, 0, 4096 * sizeof(int)));
    G53_TRY(hipMalloc((void **)&g_errs, 64 * sizeof(int)));
    G53_TRY(hipMemset(g_errs, 0, 64 * sizeof(int)));
    G53_TRY(hipHostMalloc((void **)&g_mbox, G53H_MBOX_BYTES, hipHostMallocMapped | hipHostMallocCoherent));
    memset(g_mbox, 0, G53H_MBOX_BYTES);
    G53_TRY(hipHostGetDevicePointer((void **)&g_mbox_d, g_mbox, 0));
    G53_TRY(hipHostMalloc((void **)&g_inbox, G53H_INBOX_BYTES, hipHostMallocMapped | hipHostMallocCoherent));
    memset(g_inbox, 0, G53H_INBOX_BYTES);
    G53_TRY(hipHostGetDevicePointer((void **)&g_inbox_d, g_inbox, 0));
    G53_TRY(hipDeviceSynchronize());
    if (g53_noalloc_setup(device)) return -1;
    g_device = device;
    g_ready = 1;
    return 0;
}

int g53h_current_device(void) { return g_ready ? g_device : -1; }

extern "C" int g53h_ready(void) { return g_ready ? 0 : g53h_init(0); }
extern "C" int g53h_num_cus(void) { return g_cus; }
/* Operations enqueued on the compute stream (every use of it through g53h_stream or enq counts
 * as one), and the last mailbox publication: when a wait sees that publication's sequence word
 * and nothing was enqueued after it, the stream is quiet (every kernel before it has completed). */
static unsigned long g_enq = 0, g_pub_enq = 0;
static int g_pub_slot = -1, g_quiet = 0;
static unsigned g_pub_seq = 0;
static hipStream_t enq(void)
{
    g_enq++;
    g_quiet = 0;
    return g_stream;
}
hipStream_t g53h_stream(void) { return enq(); }
void g53h_note_publish(int slot, unsigned seq)
{
    g_pub_enq = g_enq;
    g_pub_slot = slot;
    g_pub_seq = seq;
}
int g53h_quiet(void) { return g_quiet; }
hipStream_t g53h_copy_stream(void) { return g_copy; }
int *g53h_counters(void) { return g_counters; }
int *g53h_errblock(void) { return g_errs; }
unsigned *g53h_mailbox_dev(void) { return g_mbox_d; }

extern "C" void *g53h_mailbox(void) { return g53h_ready() ? nullptr : (void *)g_mbox; }
extern "C" void *g53h_inbox(void) { return g53h_ready() ? nullptr : (void *)g_inbox; }

/* 16 bytes per thread from the mapped host inbox into device memory. */
__global__ void __launch_bounds__(256) k_inbox_fetch(uint4 *__restrict__ dst, const uint4 *__restrict__ src, int n16)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n16) dst[i] = src[i];
}

extern "C" int g53h_inbox_fetch(void *dst_d, size_t off, size_t bytes)
{
    if (g53h_ready()) return -1;
    if (off % 16 || bytes % 16 || off + bytes > G53H_INBOX_BYTES || ((uintptr_t)dst_d & 15))
        return g53h_fail("g53h_inbox_fetch: %zu bytes at %zu", bytes, off);
    if (!bytes) return 0;
    const int n16 = (int)(bytes / 16);
    hipLaunchKernelGGL(k_inbox_fetch, dim3((n16 + 255) / 256), dim3(256), 0, enq(), (uint4 *)dst_d,
                       (const uint4 *)(g_inbox_d + off), n16);
    G53_LAUNCHED("k_inbox_fetch");
    return 0;
}

extern "C" int g53h_mailbox_wait(int slot, unsigned seq)
{
    if (g53h_ready()) return -1;
    if (slot < 0 || slot >= G53H_MBOX_SLOTS) return g53h_fail("g53h_mailbox_wait: slot %d", slot);
    const volatile unsigned *w = g_mbox + slot;
    /* spin while the stream works; after ~1e6 polls fall back to a blocking wait, which also
     * reports an error the stream hit (then the word never arrives) */
    const int last = slot == g_pub_slot && seq == g_pub_seq && g_enq == g_pub_enq;
    for (long i = 0; i < (1L << 20); i++)
        if (__atomic_load_n(w, __ATOMIC_ACQUIRE) == seq) {
            if (last) g_quiet = 1;
            return 0;
        }
    G53_TRY(hipStreamSynchronize(g_stream));
    if (__atomic_load_n(w, __ATOMIC_ACQUIRE) == seq) {
        if (last) g_quiet = 1;
        return 0;
    }
    return g53h_fail("g53h_mailbox_wait: slot %d never reached %u", slot, seq);
}

/* One workgroup: n bytes (a multiple of 4) from src and the G53H_NERR error words into the
 * mailbox data area at byte offset off, then the sequence word of slot. */
__global__ void __launch_bounds__(256) k_publish(unsigned *__restrict__ mb, const uint32_t *__restrict__ src, int nw,
                                                 const int *__restrict__ errs, int off_w, int slot, unsigned seq)
{
    uint32_t *d = mb + off_w;
    for (int i = threadIdx.x; i < G53H_NERR; i += 256) d[i] = (uint32_t)errs[i];
    g53_copy_words(d + G53H_NERR, src, nw, (int)threadIdx.x, 256);
    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(mb + slot, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

extern "C" int g53h_publish(int slot, unsigned seq, size_t off, const void *src_d, size_t bytes)
{
    if (g53h_ready()) return -1;
    if (slot < 0 || slot >= G53H_MBOX_SLOTS || off % 4 || bytes % 4 || off < G53H_MBOX_SLOTS * 4 ||
        off + (G53H_NERR * 4) + bytes > G53H_MBOX_BYTES)
        return g53h_fail("g53h_publish: slot %d, %zu bytes at %zu", slot, bytes, off);
    hipLaunchKernelGGL(k_publish, dim3(1), dim3(256), 0, enq(), g_mbox_d, (const uint32_t *)src_d, (int)(bytes / 4),
                       g_errs, (int)(off / 4), slot, seq);
    G53_LAUNCHED("k_publish");
    g53h_note_publish(slot, seq);
    return 0;
}

static int g_spin = 0;
extern "C" int g53h_set_spin_limit(int polls)
{
    const int old = g_spin;
    g_spin = polls > 0 ? polls : 0;
    return old;
}
int g53h_spin_limit(void) { return g_spin > 0 ? g_spin : (1 << 20); }

__global__ void k_errs_clear(int *e)
{
    if (threadIdx.x < G53H_NERR) e[threadIdx.x] = 0;
}

__global__ void k_errs_or(int *e, int word, int bits)
{
    if (threadIdx.x == 0) e[word] |= bits;
}

extern "C" int g53h_inject_errors(int word, int bits)
{
    if (g53h_ready()) return -1;
    if (word < 0 || word >= G53H_NERR) return g53h_fail("g53h_inject_errors: word %d of %d", word, G53H_NERR);
    hipLaunchKernelGGL(k_errs_or, dim3(1), dim3(64), 0, enq(), g_errs, word, bits);
    G53_LAUNCHED("k_errs_or");
    return 0;
}

extern "C" int g53h_errors_peek_async(int *host)
{
    if (g53h_ready()) return -1;
    G53_TRY(hipMemcpyAsync(host, g_errs, G53H_NERR * sizeof(int), hipMemcpyDeviceToHost, enq()));
    return 0;
}

extern "C" int g53h_errors_async(int *host)
{
    if (g53h_ready()) return -1;
    G53_TRY(hipMemcpyAsync(host, g_errs, G53H_NERR * sizeof(int), hipMemcpyDeviceToHost, enq()));
    hipLaunchKernelGGL(k_errs_clear, dim3(1), dim3(64), 0, enq(), g_errs);
    G53_LAUNCHED("k_errs_clear");
    return 0;
}

extern "C" int g53h_sync(void)
{
    if (g53h_ready()) return -1;
    G53_TRY(hipStreamSynchronize(g_stream));
    G53_TRY(hipStreamSynchronize(g_copy));
    return 0;
}

extern "C" void *g53h_alloc(size_t bytes)
{
    if (g53h_ready()) return nullptr;
    void *p = nullptr;
    if (g53h_check(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc", __FILE__, __LINE__)) return nullptr;
    return p;
}

extern "C" int g53h_free(void *p)
{
    if (!p) return 0;
    G53_TRY(hipFree(p));
    return 0;
}

extern "C" void *g53h_host_alloc(size_t bytes)
{
    if (g53h_ready()) return nullptr;
    void *p = nullptr;
    if (g53h_check(hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault), "hipHostMalloc",
                   __FILE__, __LINE__))
        return nullptr;
    return p;
}

extern "C" int g53h_host_free(void *p)
{
    if (!p) return 0;
    G53_TRY(hipHostFree(p));
    return 0;
}

extern "C" int g53h_h2d(void *dst, const void *src, size_t n)
{
    if (g53h_ready()) return -1;
    if (!n) return 0;
    G53_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, enq()));
    G53_TRY(hipStreamSynchronize(g_stream));
    return 0;
}

extern "C" int g53h_h2d_async(void *dst, const void *src, size_t n)
{
    if (g53h_ready()) return -1;
    if (!n) return 0;
    G53_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, enq()));
    return 0;
}

extern "C" int g53h_d2h(void *dst, const void *src, size_t n)
{
    if (g53h_ready()) return -1;
    if (!n) return 0;
    G53_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, enq()));
    G53_TRY(hipStreamSynchronize(g_stream));
    return 0;
}

extern "C" int g53h_d2h_async(void *dst, const void *src, size_t n)
{
    if (g53h_ready()) return -1;
    if (!n) return 0;
    G53_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, enq()));
    return 0;
}

extern "C" int g53h_d2d(void *dst, const void *src, size_t n)
{
    if (g53h_ready()) return -1;
    if (!n) return 0;
    G53_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, enq()));
    return 0;
}

extern "C" int g53h_memset(void *dst, int v, size_t n)
{
    if (g53h_ready()) return -1;
    if (!n) return 0;
    G53_TRY(hipMemsetAsync(dst, v, n, enq()));
    return 0;
}

extern "C" int g53h_is_device_ptr(const void *p)
{
    if (!p || g53h_ready()) return 0;
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();                 /* unknown pointer: plain host memory */
        return 0;
    }
    return a.type == hipMemoryTypeDevice;
}

extern "C" int g53h_mark(void)
{
    if (g53h_ready()) return -1;
    G53_TRY(hipEventRecord(g_ev[g_ev_next], enq()));
    g_ev_next ^= 1;
    return 0;
}

extern "C" float g53h_elapsed_ms(void)
{
    /* g_ev_next now points at the older mark */
    hipEvent_t a = g_ev[g_ev_next], b = g_ev[g_ev_next ^ 1];
    if (hipEventSynchronize(b) != hipSuccess) return -1.0f;
    float ms = -1.0f;
    if (hipEventElapsedTime(&ms, a, b) != hipSuccess) return -1.0f;
    return ms;
}

extern "C" int g53h_mem_info(size_t *free_b, size_t *total_b)
{
    if (g53h_ready()) return -1;
    G53_TRY(hipMemGetInfo(free_b, total_b));
    return 0;
}

void *g53h_workspace(size_t bytes)
{
    if (bytes <= g_ws_bytes) return g_ws;
    if (g_ws) {
        if (g53h_check(hipStreamSynchronize(g_stream), "hipStreamSynchronize", __FILE__, __LINE__))
            return nullptr;
        (void)hipFree(g_ws);
        g_ws = nullptr;
        g_ws_bytes = 0;
    }
    size_t want = bytes + (bytes >> 2);
    want = (want + 0xfffff) & ~(size_t)0xfffff;
    if (g53h_check(hipMalloc(&g_ws, want), "hipMalloc(workspace)", __FILE__, __LINE__)) return nullptr;
    g_ws_bytes = want;
    return g_ws;
}

/* ---------------------------------------------------------------- profiling ----
 * Per-kernel timing with HIP events on the compute stream: when enabled, the layer code
 * records an event after each kernel it launches, tagged with the kernel's id; collection
 * attributes each interval between consecutive events to the tag of the later event. */
#define G53_PROF_EVENTS 16384
static int         g_prof_on = 0;
static hipEvent_t  g_prof_ev[G53_PROF_EVENTS];
static int         g_prof_tag[G53_PROF_EVENTS];
static int         g_prof_n = 0, g_prof_made = 0;

extern "C" int g53h_prof_enable(int on)
{
    if (g53h_ready()) return -1;
    if (on && !g_prof_made) {
        for (int i = 0; i < G53_PROF_EVENTS; i++) G53_TRY(hipEventCreate(&g_prof_ev[i]));
        g_prof_made = 1;
    }
    g_prof_on = on;
    g_prof_n = 0;
    return 0;
}

void g53h_prof_mark(int tag)
{
    if (!g_prof_on || g_prof_n >= G53_PROF_EVENTS) return;
    if (hipEventRecord(g_prof_ev[g_prof_n], enq()) != hipSuccess) return;
    g_prof_tag[g_prof_n++] = tag;
}

extern "C" int g53h_prof_collect(float *ms, int *count, int ntags)
{
    if (g53h_ready()) return -1;
    for (int t = 0; t < ntags; t++) { ms[t] = 0.0f; count[t] = 0; }
    if (g_prof_n > 0) G53_TRY(hipEventSynchronize(g_prof_ev[g_prof_n - 1]));
    for (int i = 1; i < g_prof_n; i++) {
        const int tag = g_prof_tag[i];
        if (tag <= 0 || tag >= ntags) continue;      /* tag 0 opens an interval only */
        float e = 0.0f;
        G53_TRY(hipEventElapsedTime(&e, g_prof_ev[i - 1], g_prof_ev[i]));
        ms[tag] += e;
        count[tag]++;
    }
    g_prof_n = 0;
    return 0;
}
