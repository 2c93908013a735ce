/*  p2hip.hip – the device-pointer C ABI (include/p2hip.h) over the gfx950 kernels in p2hip_kernels.h.
 *
 *  Checks every shape, stride and alignment the kernels assume before launching, so a kernel never sees an operand
 *  it would index out of bounds.
 */
#include "p2hip.h"

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <climits>
#include <atomic>
#include <mutex>

#include "p2hip_kernels.h"

namespace {

thread_local char t_err[512];
thread_local hipStream_t t_stream = nullptr;

/* The allocation-free entry's workspace: one array per device, held until the process ends. Host code never passes
 * `scratch` itself to a kernel (its host-side name is not a device address): it passes the device address that
 * hipGetSymbolAddress gives for the current device, kept in g_scratch_ptr. */
constexpr size_t kScratchBytes = (size_t)P2H_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

std::once_flag g_init_once;
int g_init_rc = P2H_E_DEVICE;
char g_init_err[512];
char g_arch[64];
int g_cus = 0;
int g_wall_khz = 0;   /* rate of the constant wall clock that stream_hold reads */

int fail(int rc, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_err, sizeof t_err, fmt, ap);
    va_end(ap);
    return rc;
}

#define HIPCHK(call)                                                                                            \
    do {                                                                                                        \
        hipError_t e_ = (call);                                                                                 \
        if (e_ != hipSuccess) return fail(P2H_E_DEVICE, "%s: %s", #call, hipGetErrorString(e_));              \
    } while (0)

void load_switches();

void do_init()
{
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n < 1) {
        snprintf(g_init_err, sizeof g_init_err, "p2h_init: no HIP device (%s)", hipGetErrorString(e));
        return;
    }
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, 0);
    if (e != hipSuccess) {
        snprintf(g_init_err, sizeof g_init_err, "p2h_init: hipGetDeviceProperties: %s", hipGetErrorString(e));
        return;
    }
    snprintf(g_arch, sizeof g_arch, "%s", prop.gcnArchName);
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        snprintf(g_init_err, sizeof g_init_err, "p2h_init: device 0 is %s, this library is built for gfx950 only",
                 prop.gcnArchName);
        return;
    }
    g_cus = prop.multiProcessorCount;
    load_switches();
    if (hipDeviceGetAttribute(&g_wall_khz, hipDeviceAttributeWallClockRate, 0) != hipSuccess || g_wall_khz <= 0)
        g_wall_khz = 100000;
    e = hipSetDevice(0);
    if (e != hipSuccess) {
        snprintf(g_init_err, sizeof g_init_err, "p2h_init: hipSetDevice: %s", hipGetErrorString(e));
        return;
    }
    /* device 0's scratch address, with device 0 current (another device's is taken on its first no-alloc call) */
    void *sp = nullptr;
    if (hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)) == hipSuccess) g_scratch_ptr[0] = sp;
    g_init_rc = P2H_OK;
}

/* The device address of the current device's scratch array (taken once per device, with that device current). */
int scratch_of_current_device(void **out)
{
    int dev = 0;
    HIPCHK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(P2H_E_DEVICE, "scratch: device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        HIPCHK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(P2H_E_DEVICE, "scratch: hipGetSymbolAddress gave NULL on device %d", dev);
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return P2H_OK;
}

int ensure_init()
{
    std::call_once(g_init_once, do_init);
    if (g_init_rc != P2H_OK) return fail(g_init_rc, "%s", g_init_err);
    return P2H_OK;
}

hipStream_t stream_of(void *s)
{
    if (s) return (hipStream_t)s;
    return (hipStream_t)p2h_thread_stream();
}

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

/* an integer from the environment (tuning and comparison switches), dflt when unset or empty */
int env_int(const char *name, int dflt)
{
    const char *v = getenv(name);
    return (v && *v) ? atoi(v) : dflt;
}

/* The tuning and comparison switches, read from the environment once at initialisation and again only by
 * p2h_reload_switches: no launch reads the environment, so a host thread calling setenv races with nothing but an
 * explicit reload. kUnset marks a tile that is not forced. */
constexpr int kUnset = INT_MIN;
struct Switches {
    std::atomic<int> tile{kUnset};          /* P2H_TILE: force a five-value tile */
    std::atomic<int> split_rows{0};         /* P2H_SPLIT_ROWS: force a K split (-1: never) */
    std::atomic<int> xf_staged{1};          /* P2H_XF_STAGED: 0 loads the exact route's rows into registers */
    std::atomic<int> xf_tile{0};            /* P2H_XF_TILE: force the exact route's tile: 32 or 64 columns of 32 rows,
                                               or 1616, 1632, 1664 for 16 rows of 16, 32, 64 columns */
    std::atomic<int> exact_chain{0};        /* P2H_EXACT_CHAIN: the exact route's per-output fmaf chain */
    std::atomic<int> sgemm_any{0};          /* P2H_SGEMM_ANY: the fp32 GEMM's element loads */
    std::atomic<int> attention_fused{1};    /* P2H_ATTENTION_FUSED: 0 runs the attention as separate products */
    std::atomic<int> silu_epilogue{1};      /* P2H_SILU_EPILOGUE: 0 uses the SiLU→int8 producer in the block */
    std::atomic<int> exact_epilogue{1};     /* P2H_EXACT_EPILOGUE: 0 runs exact mode's residuals and SiLU apart */
    std::atomic<int> stack_norm_pairs{1};   /* P2H_STACK_NORM_PAIRS: 0 keeps the stack's LayerNorms unpaired */
    std::atomic<int> conv_quant{1};         /* P2H_CONV_QUANT: 0 quantises the convolution's rows apart */
    std::atomic<int> conv_tt{2};            /* P2H_CONV_TT: frames per workgroup of the quantising convolution */
    std::atomic<int> quant_rpw{0};          /* P2H_QUANT_RPW: rows per workgroup of quant_rows (1 or 4), or −4 for
                                               four waves per row (quant_rows_w4); 0: by M and K */
    std::atomic<int> dev_scope_stores{1};   /* P2H_DEVICE_SCOPE_STORES: 0 stores the five-value GEMMs' C plainly,
                                               to be written back from the L2s when the kernel ends */
    std::atomic<int> records_in_regs{1};    /* P2H_RECORDS_IN_REGISTERS: 0 streams the large-M tiles' weight records
                                               through the LDS ring with the activation rows (gemm_fv) */
    std::atomic<int> xcd_rows{-4};          /* P2H_XCD_ROWS: the small-M tiles' XCD grid rows (1, 2, 4 or 8) where the
                                               tiles divide evenly; negative: that many only where N < 4·M; 0 hands
                                               XCDs consecutive column tiles */
};
Switches g_sw;

void load_switches()
{
    const auto r = std::memory_order_relaxed;
    g_sw.tile.store(env_int("P2H_TILE", kUnset), r);
    g_sw.split_rows.store(env_int("P2H_SPLIT_ROWS", 0), r);
    g_sw.xf_staged.store(env_int("P2H_XF_STAGED", 1), r);
    g_sw.xf_tile.store(env_int("P2H_XF_TILE", 0), r);
    g_sw.exact_chain.store(env_int("P2H_EXACT_CHAIN", 0), r);
    g_sw.sgemm_any.store(env_int("P2H_SGEMM_ANY", 0), r);
    g_sw.attention_fused.store(env_int("P2H_ATTENTION_FUSED", 1), r);
    g_sw.silu_epilogue.store(env_int("P2H_SILU_EPILOGUE", 1), r);
    g_sw.exact_epilogue.store(env_int("P2H_EXACT_EPILOGUE", 1), r);
    g_sw.stack_norm_pairs.store(env_int("P2H_STACK_NORM_PAIRS", 1), r);
    g_sw.conv_quant.store(env_int("P2H_CONV_QUANT", 1), r);
    g_sw.conv_tt.store(env_int("P2H_CONV_TT", 2), r);
    g_sw.quant_rpw.store(env_int("P2H_QUANT_RPW", 0), r);
    g_sw.dev_scope_stores.store(env_int("P2H_DEVICE_SCOPE_STORES", 1), r);
    g_sw.records_in_regs.store(env_int("P2H_RECORDS_IN_REGISTERS", 1), r);
    g_sw.xcd_rows.store(env_int("P2H_XCD_ROWS", -4), r);
}

inline int switch_of(const std::atomic<int> &v) { return v.load(std::memory_order_relaxed); }
inline bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

/* Whether M rows of Y (pitch ldy floats) overlap M rows of X (pitch ldx) other than as the very same rows. */
inline bool rows_overlap(const float *dX, int ldx, const float *dY, int ldy, int M)
{
    if (dX == dY) return false;
    return (const char *)dY < (const char *)(dX + (size_t)M * ldx) &&
           (const char *)dX < (const char *)(dY + (size_t)M * ldy);
}

}  // namespace

struct P2hWeight {
    int K, N;
    const uint8_t *signs, *flags;   /* the planes, set only while the records and tables are made from them */
    const float *lo, *hi;
    uint8_t *clo;
    uint8_t *rec4;    /* 4-bit selector records, the operand of every GEMM route (fv_repack4):
                         [N/16][units][64 lanes][16 B] */
    int units;        /* 128-row K units: K rounded up / 128 */
    void *own;        /* the one device allocation this handle made */
    size_t own_bytes;
};

extern "C" {

/* ── runtime ────────────────────────────────────────────────────────────────────────────────────────────────── */

int p2h_init(void) { return ensure_init(); }

int p2h_reload_switches(void)
{
    load_switches();
    return P2H_OK;
}

const char *p2h_last_error(void) { return t_err; }

const char *p2h_device_name(void)
{
    ensure_init();
    return g_arch;
}

int p2h_device_cu_count(void)
{
    ensure_init();
    return g_cus;
}

void *p2h_stream_create(void)
{
    if (ensure_init()) return nullptr;
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) {
        fail(P2H_E_DEVICE, "hipStreamCreate failed");
        return nullptr;
    }
    return s;
}

int p2h_stream_destroy(void *stream)
{
    if (!stream) return P2H_OK;
    HIPCHK(hipStreamDestroy((hipStream_t)stream));
    return P2H_OK;
}

int p2h_stream_sync(void *stream)
{
    if (int rc = ensure_init()) return rc;
    HIPCHK(hipStreamSynchronize(stream_of(stream)));
    return P2H_OK;
}

void *p2h_thread_stream(void)
{
    if (!t_stream) {
        if (ensure_init()) return nullptr;
        if (hipStreamCreateWithFlags(&t_stream, hipStreamNonBlocking) != hipSuccess) {
            t_stream = nullptr;
            fail(P2H_E_DEVICE, "hipStreamCreate failed");
        }
    }
    return t_stream;
}

void *p2h_malloc(size_t bytes)
{
    if (ensure_init()) return nullptr;
    void *p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) {
        fail(P2H_E_NOMEM, "hipMalloc(%zu) failed", bytes);
        return nullptr;
    }
    return p;
}

int p2h_free(void *dptr)
{
    if (!dptr) return P2H_OK;
    HIPCHK(hipFree(dptr));
    return P2H_OK;
}

void *p2h_host_malloc(size_t bytes)
{
    if (ensure_init()) return nullptr;
    void *p = nullptr;
    if (hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault) != hipSuccess) {
        fail(P2H_E_NOMEM, "hipHostMalloc(%zu) failed", bytes);
        return nullptr;
    }
    return p;
}

int p2h_host_free(void *hptr)
{
    if (!hptr) return P2H_OK;
    HIPCHK(hipHostFree(hptr));
    return P2H_OK;
}

int p2h_memset(void *dptr, int value, size_t bytes, void *stream)
{
    if (int rc = ensure_init()) return rc;
    HIPCHK(hipMemsetAsync(dptr, value, bytes, stream_of(stream)));
    return P2H_OK;
}

int p2h_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream)
{
    if (int rc = ensure_init()) return rc;
    HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream_of(stream)));
    return P2H_OK;
}

int p2h_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream)
{
    if (int rc = ensure_init()) return rc;
    HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream_of(stream)));
    return P2H_OK;
}

int p2h_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream)
{
    if (int rc = ensure_init()) return rc;
    HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream_of(stream)));
    return P2H_OK;
}

int p2h_memcpy2d_h2d(void *dst, size_t dpitch, const void *src, size_t spitch, size_t row_bytes, size_t rows,
                     void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (rows == 0 || row_bytes == 0) return P2H_OK;
    if (dpitch == row_bytes && spitch == row_bytes)   /* packed rows: one linear copy (the 2-D copy goes row by row,
                                                         about 3 ms for 375 rows whatever their length) */
        HIPCHK(hipMemcpyAsync(dst, src, rows * row_bytes, hipMemcpyHostToDevice, stream_of(stream)));
    else
        HIPCHK(hipMemcpy2DAsync(dst, dpitch, src, spitch, row_bytes, rows, hipMemcpyHostToDevice, stream_of(stream)));
    return P2H_OK;
}

int p2h_memcpy2d_d2h(void *dst, size_t dpitch, const void *src, size_t spitch, size_t row_bytes, size_t rows,
                     void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (rows == 0 || row_bytes == 0) return P2H_OK;
    if (dpitch == row_bytes && spitch == row_bytes)
        HIPCHK(hipMemcpyAsync(dst, src, rows * row_bytes, hipMemcpyDeviceToHost, stream_of(stream)));
    else
        HIPCHK(hipMemcpy2DAsync(dst, dpitch, src, spitch, row_bytes, rows, hipMemcpyDeviceToHost, stream_of(stream)));
    return P2H_OK;
}

int p2h_capture_begin(void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (!stream) return fail(P2H_E_ARG, "p2h_capture_begin: capture needs an explicit stream");
    HIPCHK(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal));
    return P2H_OK;
}

int p2h_capture_end(void *stream, void **graph_exec)
{
    if (!stream || !graph_exec) return fail(P2H_E_ARG, "p2h_capture_end: NULL argument");
    hipGraph_t graph = nullptr;
    HIPCHK(hipStreamEndCapture((hipStream_t)stream, &graph));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return fail(P2H_E_DEVICE, "hipGraphInstantiate: %s", hipGetErrorString(e));
    *graph_exec = exec;
    return P2H_OK;
}

int p2h_graph_launch(void *graph_exec, void *stream)
{
    if (!graph_exec) return fail(P2H_E_ARG, "p2h_graph_launch: NULL graph");
    HIPCHK(hipGraphLaunch((hipGraphExec_t)graph_exec, stream_of(stream)));
    return P2H_OK;
}

int p2h_graph_destroy(void *graph_exec)
{
    if (!graph_exec) return P2H_OK;
    HIPCHK(hipGraphExecDestroy((hipGraphExec_t)graph_exec));
    return P2H_OK;
}

void *p2h_event_create(void)
{
    if (ensure_init()) return nullptr;
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) {
        fail(P2H_E_DEVICE, "hipEventCreate failed");
        return nullptr;
    }
    return e;
}

int p2h_event_destroy(void *event)
{
    if (!event) return P2H_OK;
    HIPCHK(hipEventDestroy((hipEvent_t)event));
    return P2H_OK;
}

int p2h_event_record(void *event, void *stream)
{
    if (int rc = ensure_init()) return rc;
    HIPCHK(hipEventRecord((hipEvent_t)event, stream_of(stream)));
    return P2H_OK;
}

int p2h_event_sync(void *event)
{
    HIPCHK(hipEventSynchronize((hipEvent_t)event));
    return P2H_OK;
}

int p2h_stream_wait_event(void *stream, void *event)
{
    if (int rc = ensure_init()) return rc;
    if (!event) return fail(P2H_E_ARG, "p2h_stream_wait_event: NULL event");
    HIPCHK(hipStreamWaitEvent(stream_of(stream), (hipEvent_t)event, 0));
    return P2H_OK;
}

int p2h_stream_hold(void *stream, unsigned usec)
{
    if (int rc = ensure_init()) return rc;
    if (usec > 1000000u) return fail(P2H_E_ARG, "p2h_stream_hold: %u us is above the 1 s limit", usec);
    const unsigned long long ticks = (unsigned long long)usec * (unsigned long long)g_wall_khz / 1000ull;
    /* a nap is at least 8k cycles, i.e. over 2 us at any clock this device runs: usec/2 + 16 naps bound the wait */
    hipLaunchKernelGGL(p2k::stream_hold, dim3(1), dim3(64), 0, stream_of(stream), ticks, usec / 2u + 16u);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

float p2h_event_elapsed_ms(void *start, void *stop)
{
    float ms = -1.0f;
    if (hipEventElapsedTime(&ms, (hipEvent_t)start, (hipEvent_t)stop) != hipSuccess) return -1.0f;
    return ms;
}

/* ── weights ────────────────────────────────────────────────────────────────────────────────────────────────── */

static P2hWeight *weight_new(int K, int N, bool copy_planes)
{
    if (K < 0 || N <= 0 || N % 16 != 0) {
        fail(P2H_E_ARG, "five-value weight: N = %d must be a positive multiple of 16 (K = %d)", N, K);
        return nullptr;
    }
    size_t off_lo = 0, off_hi = 0, off = 0;
    if (copy_planes) {   /* lo and hi stay (the exact route reads them); the sign and flag planes do not */
        off_lo = off; off += align_up((size_t)N * 4, 256);
        off_hi = off; off += align_up((size_t)N * 4, 256);
    }
    size_t off_clo = off; off += align_up((size_t)N, 256);
    const int units = (K + 127) / 128;
    size_t off_rec4 = off; off += align_up((size_t)(N / 16) * units * 1024 + 16, 256);
    void *base = nullptr;
    if (hipMalloc(&base, off) != hipSuccess) {
        fail(P2H_E_NOMEM, "five-value weight: hipMalloc(%zu) failed", off);
        return nullptr;
    }
    P2hWeight *w = new P2hWeight();
    w->K = K; w->N = N;
    uint8_t *b = (uint8_t *)base;
    if (copy_planes) {
        w->lo = (const float *)(b + off_lo);
        w->hi = (const float *)(b + off_hi);
    }
    w->clo = b + off_clo;
    w->rec4 = b + off_rec4;
    w->units = units;
    w->own = base;
    w->own_bytes = off;
    return w;
}

static int weight_tables(P2hWeight *w)
{
    hipStream_t s = stream_of(nullptr);
    hipLaunchKernelGGL(p2k::fv_tables, dim3((w->N + 255) / 256), dim3(256), 0, s, w->N, w->lo, w->hi, w->clo);
    HIPCHK(hipGetLastError());
    const size_t recs = (size_t)(w->N / 16) * w->units * 64;
    if (recs > 0) {
        hipLaunchKernelGGL(p2k::fv_repack4, dim3((unsigned)((recs + 255) / 256)), dim3(256), 0, s, w->K, w->N,
                           w->units, w->signs, w->flags, (uint4 *)w->rec4);
        HIPCHK(hipGetLastError());
    }
    HIPCHK(hipStreamSynchronize(s));
    return P2H_OK;
}

P2hWeight *p2h_fv_weight_upload(const unsigned char *signs, const unsigned char *flags, const float *lo,
                                const float *hi, int K, int N)
{
    if (ensure_init()) return nullptr;
    if (!signs || !flags || !lo || !hi) {
        fail(P2H_E_ARG, "p2h_fv_weight_upload: NULL plane");
        return nullptr;
    }
    P2hWeight *w = weight_new(K, N, true);
    if (!w) return nullptr;
    /* the planes only pass through the device: a staging buffer the records and tables are made from, freed once
     * they are (the device copy keeps 0.5 byte per weight, the records, against 0.875 with the planes kept) */
    size_t kn = (size_t)K * N;
    const size_t sb = align_up(kn / 4 ? kn / 4 : 1, 256), fb = align_up(kn / 8 ? kn / 8 : 1, 256);
    void *stage = nullptr;
    if (hipMalloc(&stage, sb + fb) != hipSuccess) {
        fail(P2H_E_NOMEM, "p2h_fv_weight_upload: hipMalloc(%zu) for the planes failed", sb + fb);
        p2h_weight_free(w);
        return nullptr;
    }
    w->signs = (const uint8_t *)stage;
    w->flags = (const uint8_t *)stage + sb;
    hipStream_t s = stream_of(nullptr);
    bool ok = hipMemcpyAsync((void *)w->signs, signs, kn / 4, hipMemcpyHostToDevice, s) == hipSuccess &&
              hipMemcpyAsync((void *)w->flags, flags, kn / 8, hipMemcpyHostToDevice, s) == hipSuccess &&
              hipMemcpyAsync((void *)w->lo, lo, (size_t)N * 4, hipMemcpyHostToDevice, s) == hipSuccess &&
              hipMemcpyAsync((void *)w->hi, hi, (size_t)N * 4, hipMemcpyHostToDevice, s) == hipSuccess;
    const int rc = ok ? weight_tables(w) : fail(P2H_E_DEVICE, "p2h_fv_weight_upload: copy failed");
    if (!ok) (void)hipStreamSynchronize(s);   /* no copy may still read host memory or write the staging buffer */
    (void)hipFree(stage);                      /* weight_tables synchronised: nothing reads the planes any more */
    w->signs = w->flags = nullptr;
    if (rc != P2H_OK) {
        p2h_weight_free(w);
        return nullptr;
    }
    return w;
}

P2hWeight *p2h_fv_weight_wrap(const void *d_signs, const void *d_flags, const float *d_lo, const float *d_hi,
                              int K, int N)
{
    if (ensure_init()) return nullptr;
    if (!d_signs || !d_flags || !d_lo || !d_hi || !aligned(d_signs, 4) || !aligned(d_flags, 2) ||
        !aligned(d_lo, 4) || !aligned(d_hi, 4)) {
        fail(P2H_E_ARG, "p2h_fv_weight_wrap: planes must be non-NULL, signs 4-byte and flags 2-byte aligned");
        return nullptr;
    }
    P2hWeight *w = weight_new(K, N, false);
    if (!w) return nullptr;
    w->signs = (const uint8_t *)d_signs;
    w->flags = (const uint8_t *)d_flags;
    w->lo = d_lo;
    w->hi = d_hi;
    const int rc = weight_tables(w);
    w->signs = w->flags = nullptr;   /* every kernel reads the records: the caller's planes are not needed again */
    if (rc != P2H_OK) {
        p2h_weight_free(w);
        return nullptr;
    }
    return w;
}

void p2h_weight_free(P2hWeight *w)
{
    if (!w) return;
    if (w->own) (void)hipFree(w->own);
    delete w;
}

int p2h_weight_shape(const P2hWeight *w, int *K, int *N)
{
    if (!w) return fail(P2H_E_ARG, "NULL weight");
    if (K) *K = w->K;
    if (N) *N = w->N;
    return P2H_OK;
}

size_t p2h_weight_device_bytes(const P2hWeight *w) { return w ? w->own_bytes : 0; }

int p2h_fv_pack_codes(const P2hWeight *w, signed char *d_codes, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (!w || !d_codes) return fail(P2H_E_ARG, "p2h_fv_pack_codes: NULL argument");
    if (w->K % 4 != 0) return fail(P2H_E_ARG, "p2h_fv_pack_codes: K = %d is not a multiple of 4", w->K);
    if (!aligned(d_codes, 4)) return fail(P2H_E_ARG, "p2h_fv_pack_codes: output must be 4-byte aligned");
    size_t total = (size_t)(w->N / 16) * (w->K / 4) * 16;
    if (total == 0) return P2H_OK;
    hipLaunchKernelGGL(p2k::fv_pack_codes, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream_of(stream),
                       w->K, w->N, w->units, w->rec4, w->clo, (uint32_t *)d_codes);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

/* ── activations ────────────────────────────────────────────────────────────────────────────────────────────── */

int p2h_q_ld(int K) { return (int)align_up((size_t)(K > 0 ? K : 0), P2H_Q_KALIGN); }

size_t p2h_q_bytes(int M, int K)
{
    if (M <= 0 || K <= 0) return 0;
    return align_up((size_t)M, 16) * (size_t)p2h_q_ld(K);
}

int p2h_quant_rows(int M, int K, const float *dA, int lda, signed char *dQ, int ldq, float *dScales, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (M < 0 || K < 0 || K % 4 != 0) return fail(P2H_E_ARG, "p2h_quant_rows: K = %d must be a multiple of 4", K);
    if (M == 0) return P2H_OK;
    if (!dA || !dQ || !dScales || lda < K) return fail(P2H_E_ARG, "p2h_quant_rows: bad pointer or lda");
    if (ldq < p2h_q_ld(K) || ldq % P2H_Q_KALIGN != 0 || !aligned(dQ, 16))
        return fail(P2H_E_ARG, "p2h_quant_rows: ldq = %d must be >= %d and a multiple of %d, Q 16-byte aligned",
                    ldq, p2h_q_ld(K), P2H_Q_KALIGN);
    const int vec_ok = (lda % 4 == 0) && aligned(dA, 16);
    const int Mp = (int)align_up((size_t)M, 16);
    /* one row per workgroup where that leaves most CUs a row at most (M <= 192): a workgroup of four rows reads four
     * rows' bytes on one CU (measured at K = 4096: M = 38 2.91 against 3.49 µs, M = 160 3.27 against 3.55; at M = 375
     * four rows per workgroup win, 3.72 against 4.24) */
    const int forced_rpw = switch_of(g_sw.quant_rpw);
    const int rpw = forced_rpw == 1 || forced_rpw == 4 ? forced_rpw : (Mp <= 192 ? 1 : 4);
    const dim3 grid((unsigned)((Mp + rpw - 1) / rpw)), block(64 * rpw);
    hipStream_t s = stream_of(stream);
    /* four waves per row for a few long rows (K = 4096: M = 38 2.56 against 2.94 µs, M = 9 2.43 against 2.86, M = 250
     * 3.38 against 3.62; at M = 375 one wave per row wins, 3.69 against 4.01, and at K = 1024 for every M); forced with
     * P2H_QUANT_RPW = -4 */
    const bool w4 = forced_rpw == -4 || (forced_rpw == 0 && Mp <= 256 && ldq >= 4096);
    if (w4 && ldq <= 8192) {
        auto launch4 = [&](auto nch_tag, auto vec_tag) {
            hipLaunchKernelGGL((p2k::quant_rows_w4<decltype(nch_tag)::value, decltype(vec_tag)::value>),
                               dim3((unsigned)Mp), dim3(256), 0, s, M, Mp, K, dA, lda, (int8_t *)dQ, ldq, dScales);
        };
        auto by_width4 = [&](auto vec_tag) {
            if (ldq <= 4096) launch4(std::integral_constant<int, 1>{}, vec_tag);
            else launch4(std::integral_constant<int, 2>{}, vec_tag);
        };
        if (vec_ok) by_width4(std::true_type{});
        else by_width4(std::false_type{});
        HIPCHK(hipGetLastError());
        return P2H_OK;
    }
    auto launch = [&](auto nch_tag, auto vec_tag) {
        constexpr int NCH = decltype(nch_tag)::value;
        constexpr bool VEC = decltype(vec_tag)::value;
        if (rpw == 1)
            hipLaunchKernelGGL((p2k::quant_rows<NCH, VEC, 1>), grid, block, 0, s, M, Mp, K, dA, lda, (int8_t *)dQ,
                               ldq, dScales);
        else
            hipLaunchKernelGGL((p2k::quant_rows<NCH, VEC, 4>), grid, block, 0, s, M, Mp, K, dA, lda, (int8_t *)dQ,
                               ldq, dScales);
    };
    auto by_width = [&](auto vec_tag) {
        switch ((ldq + 1023) / 1024) {   /* row chunks per lane kept in registers (0: the row is read twice) */
        case 1: launch(std::integral_constant<int, 1>{}, vec_tag); break;
        case 2: launch(std::integral_constant<int, 2>{}, vec_tag); break;
        case 3: launch(std::integral_constant<int, 3>{}, vec_tag); break;
        case 4: launch(std::integral_constant<int, 4>{}, vec_tag); break;
        default: launch(std::integral_constant<int, 0>{}, vec_tag); break;
        }
    };
    if (vec_ok) by_width(std::true_type{});
    else by_width(std::false_type{});
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

/* ── self-checks ────────────────────────────────────────────────────────────────────────────────────────────── */

int p2h_recip_selftest(unsigned long long *result3)
{
    if (int rc = ensure_init()) return rc;
    if (!result3) return fail(P2H_E_ARG, "p2h_recip_selftest: null result");
    unsigned long long init[3] = {0ull, ~0ull, 0ull}, *d = nullptr;
    HIPCHK(hipMalloc(&d, sizeof init));
    hipError_t e = hipMemcpy(d, init, sizeof init, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(p2k::recip_check, dim3(8192), dim3(256), 0, 0, 0x3F800000u, 0x7E800000u, d);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(result3, d, sizeof init, hipMemcpyDeviceToHost);
    hipFree(d);
    if (e != hipSuccess) return fail(P2H_E_DEVICE, "p2h_recip_selftest: %s", hipGetErrorString(e));
    return P2H_OK;
}

/* ── producers ──────────────────────────────────────────────────────────────────────────────────────────────── */

/* Checks shared by the four producers, then one produce_rows launch over the padded rows [0, roundup(M, 16)). */
static int produce(const char *name, int kind, p2k::ProdArgs a, bool vec, hipStream_t s)
{
    if (a.M < 0 || a.K < 0 || (a.M > 0 && a.K == 0) || a.K > P2H_PROD_KMAX)
        return fail(P2H_E_ARG, "%s: %d rows of %d columns (columns 1..%d)", name, a.M, a.K, P2H_PROD_KMAX);
    if (a.M == 0) return P2H_OK;
    if (a.Y) {   /* fp32 rows: the row length picks the kernel's chunks as a quantised row's pitch would */
        if (!a.X || a.ldy < a.K) return fail(P2H_E_ARG, "%s: null input or ldy < %d", name, a.K);
        a.ldq = p2h_q_ld(a.K);
    } else {
        if (!a.X || !a.Q || !a.scales) return fail(P2H_E_ARG, "%s: null pointer", name);
        if (a.ldq < p2h_q_ld(a.K) || a.ldq % P2H_Q_KALIGN != 0 || a.ldq > P2H_PROD_KMAX || !aligned(a.Q, 16))
            return fail(P2H_E_ARG, "%s: ldq = %d must be >= %d, <= %d and a multiple of %d, Q 16-byte aligned", name,
                        a.ldq, p2h_q_ld(a.K), P2H_PROD_KMAX, P2H_Q_KALIGN);
    }
    a.Mp = (int)align_up((size_t)a.M, 16);
    if (kind == p2k::PROD_CMAJOR && !a.Y && a.K <= 1024 && a.ldq <= 1024) {   /* 16 rows per workgroup via LDS */
        hipLaunchKernelGGL(p2k::cmajor_tile, dim3((unsigned)align_up((size_t)(a.Mp / 16), 16)), dim3(1024), 0, s, a);
        HIPCHK(hipGetLastError());
        return P2H_OK;
    }
    /* rows longer than 1024 when there are too few of them to give every CU a workgroup of four rows (not
     * LayerNorm, whose sums run on one wave): a workgroup of four waves per row. Measured: SiLU over 375 rows of
     * 4096, 6.4 -> 5.5 us; over 6000 rows one wave per row stays faster. */
    const int cus = g_cus > 0 ? g_cus : 256;
    const bool wide = kind != p2k::PROD_LN && a.K > 1024 && (a.Mp + 3) / 4 < cus;
    const dim3 grid((unsigned)(wide ? a.Mp : (a.Mp + 3) / 4)), block(256);
    const bool ln_regs = a.Mp <= 2048;   /* LayerNorm's sums from registers when the rows are few */
    auto launch = [&](auto kind_tag, auto nch_tag, auto vec_tag) {
        constexpr int KIND = decltype(kind_tag)::value;
        if constexpr (KIND != p2k::PROD_LN) {
            if (wide) {   /* ldq <= 4096: one chunk per lane */
                hipLaunchKernelGGL((p2k::produce_rows<KIND, 1, decltype(vec_tag)::value, 4>), grid, block, 0, s, a);
                return;
            }
        } else if constexpr (decltype(nch_tag)::value == 1) {
            if (ln_regs) {
                hipLaunchKernelGGL((p2k::produce_rows<KIND, 1, decltype(vec_tag)::value, 1, true>), grid, block, 0, s,
                                   a);
                return;
            }
        }
        hipLaunchKernelGGL((p2k::produce_rows<KIND, decltype(nch_tag)::value, decltype(vec_tag)::value>), grid, block,
                           0, s, a);
    };
    auto by_width = [&](auto kind_tag, auto vec_tag) {
        switch (wide ? 1 : (a.ldq + 1023) / 1024) {   /* 16-column chunks per lane, the row kept in registers */
        case 1: launch(kind_tag, std::integral_constant<int, 1>{}, vec_tag); break;
        case 2: launch(kind_tag, std::integral_constant<int, 2>{}, vec_tag); break;
        case 3: launch(kind_tag, std::integral_constant<int, 3>{}, vec_tag); break;
        default: launch(kind_tag, std::integral_constant<int, 4>{}, vec_tag); break;
        }
    };
    auto by_vec = [&](auto kind_tag) {
        if (vec) by_width(kind_tag, std::true_type{});
        else by_width(kind_tag, std::false_type{});
    };
    switch (kind) {
    case p2k::PROD_SILU: by_vec(std::integral_constant<int, p2k::PROD_SILU>{}); break;
    case p2k::PROD_LN: by_vec(std::integral_constant<int, p2k::PROD_LN>{}); break;
    case p2k::PROD_HEADS: by_vec(std::integral_constant<int, p2k::PROD_HEADS>{}); break;
    default: by_width(std::integral_constant<int, p2k::PROD_CMAJOR>{}, std::false_type{}); break;
    }
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

int p2h_layer_norm_quant_rows(int M, int D, const float *dX, int ldx, const float *dGamma, const float *dBeta,
                              signed char *dQ, int ldq, float *dScales, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (M > 0 && (ldx < D || !dGamma || !dBeta))
        return fail(P2H_E_ARG, "p2h_layer_norm_quant_rows: ldx = %d < D = %d or null gamma / beta", ldx, D);
    p2k::ProdArgs a{};
    a.M = M; a.K = D; a.X = dX; a.ldx = ldx; a.gamma = dGamma; a.beta = dBeta;
    a.Q = (int8_t *)dQ; a.ldq = ldq; a.scales = dScales;
    return produce("p2h_layer_norm_quant_rows", p2k::PROD_LN, a,
                   D % 4 == 0 && ldx % 4 == 0 && aligned(dX, 16) && aligned(dGamma, 16) && aligned(dBeta, 16),
                   stream_of(stream));
}

int p2h_layer_norm2_quant_rows(int M, int D, const float *dX, int ldx, const float *dGamma1, const float *dBeta1,
                               float *dY, int ldy, const float *dGamma2, const float *dBeta2, signed char *dQ, int ldq,
                               float *dScales, void *stream)
{
    /* the arguments first, so that they fail the same way with or without a device */
    const char *name = "p2h_layer_norm2_quant_rows";
    if (M < 0 || D < 1 || D > 1024) return fail(P2H_E_ARG, "%s: %d rows of %d columns (columns 1..1024)", name, M, D);
    if (M == 0) return P2H_OK;
    if (!dX || !dY || !dGamma1 || !dBeta1 || !dGamma2 || !dBeta2 || !dQ || !dScales || ldx < D || ldy < D)
        return fail(P2H_E_ARG, "%s: null pointer, or ldx = %d / ldy = %d < D = %d", name, ldx, ldy, D);
    /* Y may be X itself (each wave reads its whole row before writing it), but not part of other rows of X: a
     * wave's stores would land in rows another wave has not read yet */
    if (rows_overlap(dX, ldx, dY, ldy, M))
        return fail(P2H_E_ARG, "%s: X and Y overlap without being the same rows", name);
    if (dX == dY && ldx != ldy) return fail(P2H_E_ARG, "%s: in place needs ldy == ldx", name);
    if (ldq < p2h_q_ld(D) || ldq % P2H_Q_KALIGN != 0 || ldq > 1024 || !aligned(dQ, 16))
        return fail(P2H_E_ARG, "%s: ldq = %d must be >= %d, <= 1024 and a multiple of %d, Q 16-byte aligned", name,
                    ldq, p2h_q_ld(D), P2H_Q_KALIGN);
    if (int rc = ensure_init()) return rc;
    p2k::ProdArgs a{};
    a.M = M; a.K = D; a.X = dX; a.ldx = ldx; a.gamma = dGamma1; a.beta = dBeta1;
    a.gamma2 = dGamma2; a.beta2 = dBeta2; a.Y1 = dY; a.ldy1 = ldy;
    a.Q = (int8_t *)dQ; a.ldq = ldq; a.scales = dScales;
    a.Mp = (int)align_up((size_t)M, 16);
    const bool vec = D % 4 == 0 && ldx % 4 == 0 && aligned(dX, 16) && aligned(dGamma1, 16) && aligned(dBeta1, 16);
    const dim3 grid((unsigned)((a.Mp + 3) / 4)), block(256);
    hipStream_t s = stream_of(stream);
    const bool regs = a.Mp <= 2048;   /* as p2h_layer_norm_quant_rows: the sums from registers when rows are few */
    using p2k::produce_rows;
    constexpr int LN = p2k::PROD_LN;
    if (vec && regs) hipLaunchKernelGGL((produce_rows<LN, 1, true, 1, true, true>), grid, block, 0, s, a);
    else if (vec) hipLaunchKernelGGL((produce_rows<LN, 1, true, 1, false, true>), grid, block, 0, s, a);
    else if (regs) hipLaunchKernelGGL((produce_rows<LN, 1, false, 1, true, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((produce_rows<LN, 1, false, 1, false, true>), grid, block, 0, s, a);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

int p2h_silu_quant_rows(int M, int K, const float *dH, int ldh, signed char *dQ, int ldq, float *dScales, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (K % 8 != 0) return fail(P2H_E_ARG, "p2h_silu_quant_rows: K = %d must be a multiple of 8", K);
    if (M > 0 && ldh < K) return fail(P2H_E_ARG, "p2h_silu_quant_rows: ldh = %d < K = %d", ldh, K);
    p2k::ProdArgs a{};
    a.M = M; a.K = K; a.X = dH; a.ldx = ldh; a.Q = (int8_t *)dQ; a.ldq = ldq; a.scales = dScales;
    return produce("p2h_silu_quant_rows", p2k::PROD_SILU, a, ldh % 4 == 0 && aligned(dH, 16), stream_of(stream));
}

int p2h_concat_heads_quant_rows(int H, int T, int Dh, const float *dAttnH, signed char *dQ, int ldq, float *dScales,
                                void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (H < 0 || Dh < 0 || (long long)H * Dh > P2H_PROD_KMAX)
        return fail(P2H_E_ARG, "p2h_concat_heads_quant_rows: H = %d, Dh = %d (H·Dh <= %d)", H, Dh, P2H_PROD_KMAX);
    p2k::ProdArgs a{};
    a.M = T; a.K = H * Dh; a.X = dAttnH; a.T = T; a.Dh = Dh; a.Q = (int8_t *)dQ; a.ldq = ldq; a.scales = dScales;
    return produce("p2h_concat_heads_quant_rows", p2k::PROD_HEADS, a, Dh % 16 == 0 && aligned(dAttnH, 16),
                   stream_of(stream));
}

int p2h_channel_major_quant_rows(int D, int T, const float *dDW, signed char *dQ, int ldq, float *dScales, void *stream)
{
    if (int rc = ensure_init()) return rc;
    p2k::ProdArgs a{};
    a.M = T; a.K = D; a.X = dDW; a.T = T; a.Q = (int8_t *)dQ; a.ldq = ldq; a.scales = dScales;
    return produce("p2h_channel_major_quant_rows", p2k::PROD_CMAJOR, a, false, stream_of(stream));
}

int p2h_layer_norm_rows(int M, int D, const float *dX, int ldx, const float *dGamma, const float *dBeta, float *dY,
                        int ldy, void *stream)
{
    /* the arguments first, so that they fail the same way with or without a device */
    if (M > 0 && (ldx < D || !dGamma || !dBeta || !dY))
        return fail(P2H_E_ARG, "p2h_layer_norm_rows: ldx = %d < D = %d or a null pointer", ldx, D);
    if (M > 0 && rows_overlap(dX, ldx, dY, ldy, M))
        return fail(P2H_E_ARG, "p2h_layer_norm_rows: X and Y overlap without being the same rows");
    if (M > 0 && dX == dY && ldx != ldy) return fail(P2H_E_ARG, "p2h_layer_norm_rows: in place needs ldy == ldx");
    if (int rc = ensure_init()) return rc;
    p2k::ProdArgs a{};
    a.M = M; a.K = D; a.X = dX; a.ldx = ldx; a.gamma = dGamma; a.beta = dBeta; a.Y = dY; a.ldy = ldy;
    return produce("p2h_layer_norm_rows", p2k::PROD_LN, a,
                   D % 4 == 0 && ldx % 4 == 0 && aligned(dX, 16) && aligned(dGamma, 16) && aligned(dBeta, 16),
                   stream_of(stream));
}

int p2h_concat_heads_rows(int T, const float *dAttnH, float *dY, void *stream)
{
    if (int rc = ensure_init()) return rc;
    p2k::ProdArgs a{};
    a.M = T; a.K = p2k::kD; a.X = dAttnH; a.T = T; a.Dh = p2k::kDh; a.Y = dY; a.ldy = p2k::kD;
    return produce("p2h_concat_heads_rows", p2k::PROD_HEADS, a, aligned(dAttnH, 16), stream_of(stream));
}

int p2h_channel_major_rows(int T, const float *dDW, float *dY, void *stream)
{
    if (int rc = ensure_init()) return rc;
    p2k::ProdArgs a{};
    a.M = T; a.K = p2k::kD; a.X = dDW; a.T = T; a.Y = dY; a.ldy = p2k::kD;
    return produce("p2h_channel_major_rows", p2k::PROD_CMAJOR, a, false, stream_of(stream));
}

/* ── the conformer block between its linears ─────────────────────────────────────────────────────────────────── */

static unsigned blocks_of(size_t n) { return (unsigned)((n + 255) / 256); }

int p2h_gather_heads(int T, const float *dQKV, const float *dBiasU, const float *dBiasV, float *dQu, float *dQv,
                     float *dKt, float *dVh, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (T < 0) return fail(P2H_E_ARG, "p2h_gather_heads: T = %d", T);
    if (T == 0) return P2H_OK;
    if (!dQKV || !dBiasU || !dBiasV || !dQu || !dQv || !dKt || !dVh)
        return fail(P2H_E_ARG, "p2h_gather_heads: null pointer");
    hipStream_t s = stream_of(stream);
    hipLaunchKernelGGL(p2k::gather_qv, dim3(blocks_of((size_t)T * p2k::kD)), dim3(256), 0, s, T, dQKV, dBiasU,
                       dBiasV, dQu, dQv, dVh);
    hipLaunchKernelGGL(p2k::head_transpose, dim3((unsigned)((T + 31) / 32), p2k::kH), dim3(256), 0, s, T,
                       dQKV + p2k::kD, 3 * p2k::kD, dKt);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

int p2h_transpose_pos(int L, const float *dP, float *dPt, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (L < 0) return fail(P2H_E_ARG, "p2h_transpose_pos: L = %d", L);
    if (L == 0) return P2H_OK;
    if (!dP || !dPt) return fail(P2H_E_ARG, "p2h_transpose_pos: null pointer");
    hipLaunchKernelGGL(p2k::head_transpose, dim3((unsigned)((L + 31) / 32), p2k::kH), dim3(256), 0, stream_of(stream),
                       L, dP, p2k::kD, dPt);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

int p2h_combine_softmax(int T, float *dAC, const float *dBD, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (T < 0) return fail(P2H_E_ARG, "p2h_combine_softmax: T = %d", T);
    if (T == 0) return P2H_OK;
    if (!dAC || !dBD) return fail(P2H_E_ARG, "p2h_combine_softmax: null pointer");
    const int rows = p2k::kH * T;
    const float scale = 1.0f / sqrtf((float)p2k::kDh);   /* encoder.c:521; correctly rounded, as GCC folds it */
    hipStream_t s = stream_of(stream);
    const dim3 wgrid((unsigned)((rows + 3) / 4));   /* one wave per row while the row fits its registers */
    if (T <= 64 * 6) hipLaunchKernelGGL(p2k::combine_softmax_wave<6>, wgrid, dim3(256), 0, s, rows, T, scale, dAC, dBD);
    else if (T <= 64 * 12)
        hipLaunchKernelGGL(p2k::combine_softmax_wave<12>, wgrid, dim3(256), 0, s, rows, T, scale, dAC, dBD);
    else if (T <= 64 * 32)
        hipLaunchKernelGGL(p2k::combine_softmax_wave<32>, wgrid, dim3(256), 0, s, rows, T, scale, dAC, dBD);
    else
        hipLaunchKernelGGL(p2k::combine_softmax_rows, dim3((unsigned)((rows + 31) / 32)), dim3(256), 0, s, rows, T,
                           scale, dAC, dBD);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

static int attention(int T, const float *dQKV, const float *dBiasU, const float *dBiasV, const float *dP,
                     float *dAttnH, int rows, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (T < 0 || T > P2H_ATTENTION_TMAX)
        return fail(P2H_E_ARG, "p2h_attention: T = %d (1 .. %d)", T, P2H_ATTENTION_TMAX);
    if (T == 0) return P2H_OK;
    if (!dQKV || !dBiasU || !dBiasV || !dP || !dAttnH) return fail(P2H_E_ARG, "p2h_attention: null pointer");
    if (!aligned(dQKV, 16) || !aligned(dBiasU, 16) || !aligned(dBiasV, 16) || !aligned(dP, 16) || !aligned(dAttnH, 16))
        return fail(P2H_E_ARG, "p2h_attention: operands must be 16-byte aligned");
    const float scale = 1.0f / sqrtf((float)p2k::kDh);   /* encoder.c:521 */
    const dim3 grid((unsigned)(p2k::kH * ((T + 15) / 16)));
    hipStream_t s = stream_of(stream);
    if (T <= 64 * 6)
        hipLaunchKernelGGL(p2k::attention_rel<6>, grid, dim3(512), 0, s, T, scale, dQKV, dBiasU, dBiasV, dP, dAttnH, rows);
    else
        hipLaunchKernelGGL(p2k::attention_rel<12>, grid, dim3(512), 0, s, T, scale, dQKV, dBiasU, dBiasV, dP, dAttnH,
                           rows);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

int p2h_attention_heads(int T, const float *dQKV, const float *dBiasU, const float *dBiasV, const float *dP,
                        float *dAttnH, void *stream)
{
    return attention(T, dQKV, dBiasU, dBiasV, dP, dAttnH, 0, stream);
}

int p2h_attention_rows(int T, const float *dQKV, const float *dBiasU, const float *dBiasV, const float *dP,
                       float *dAttn, void *stream)
{
    return attention(T, dQKV, dBiasU, dBiasV, dP, dAttn, 1, stream);
}

int p2h_glu_channel_major(int T, const float *dPW1, float *dGated, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (T < 0) return fail(P2H_E_ARG, "p2h_glu_channel_major: T = %d", T);
    if (T == 0) return P2H_OK;
    if (!dPW1 || !dGated) return fail(P2H_E_ARG, "p2h_glu_channel_major: null pointer");
    hipLaunchKernelGGL(p2k::glu_channel_major, dim3((unsigned)((T + 31) / 32), p2k::kD / 64), dim3(256), 0,
                       stream_of(stream), T, dPW1, dGated);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

int p2h_depthwise_conv_silu(int T, const float *dGated, const float *dW, const float *dB, float *dOut, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (T < 0) return fail(P2H_E_ARG, "p2h_depthwise_conv_silu: T = %d", T);
    if (T == 0) return P2H_OK;
    if (!dGated || !dW || !dB || !dOut) return fail(P2H_E_ARG, "p2h_depthwise_conv_silu: null pointer");
    if (dGated == dOut) return fail(P2H_E_ARG, "p2h_depthwise_conv_silu: in place is not supported");
    hipLaunchKernelGGL(p2k::dwconv_silu, dim3((unsigned)((T + 255) / 256), p2k::kD), dim3(256), 0, stream_of(stream),
                       T, dGated, dW, dB, dOut);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

int p2h_glu_depthwise_conv_silu(int T, const float *dPW1, const float *dW, const float *dB, float *dOut,
                                void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (T < 0) return fail(P2H_E_ARG, "p2h_glu_depthwise_conv_silu: T = %d", T);
    if (T == 0) return P2H_OK;
    if (!dPW1 || !dW || !dB || !dOut) return fail(P2H_E_ARG, "p2h_glu_depthwise_conv_silu: null pointer");
    hipLaunchKernelGGL(p2k::glu_dwconv_silu<false>, dim3((unsigned)((T + 31) / 32), p2k::kD / 16), dim3(256), 0,
                       stream_of(stream), T, dPW1, dW, dB, dOut);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

int p2h_glu_depthwise_conv_silu_rows(int T, const float *dPW1, const float *dW, const float *dB, float *dOut,
                                     void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (T < 0) return fail(P2H_E_ARG, "p2h_glu_depthwise_conv_silu_rows: T = %d", T);
    if (T == 0) return P2H_OK;
    if (!dPW1 || !dW || !dB || !dOut) return fail(P2H_E_ARG, "p2h_glu_depthwise_conv_silu_rows: null pointer");
    hipLaunchKernelGGL(p2k::glu_dwconv_silu<true>, dim3((unsigned)((T + 31) / 32), p2k::kD / 16), dim3(256), 0,
                       stream_of(stream), T, dPW1, dW, dB, dOut);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

int p2h_glu_depthwise_conv_silu_quant_rows(int T, const float *dPW1, const float *dW, const float *dB,
                                           signed char *dQ, int ldq, float *dScales, void *stream)
{
    if (int rc = ensure_init()) return rc;
    const char *name = "p2h_glu_depthwise_conv_silu_quant_rows";
    if (T < 0) return fail(P2H_E_ARG, "%s: T = %d", name, T);
    if (T == 0) return P2H_OK;
    if (!dPW1 || !dW || !dB || !dQ || !dScales) return fail(P2H_E_ARG, "%s: null pointer", name);
    if (ldq < p2h_q_ld(p2k::kD) || ldq % P2H_Q_KALIGN != 0 || !aligned(dQ, 16))
        return fail(P2H_E_ARG, "%s: ldq = %d must be >= %d and a multiple of %d, Q 16-byte aligned", name, ldq,
                    p2h_q_ld(p2k::kD), P2H_Q_KALIGN);
    const int tt = switch_of(g_sw.conv_tt);
    hipStream_t s = stream_of(stream);
    auto go = [&](auto kern, int TT) {
        hipLaunchKernelGGL(kern, dim3((unsigned)((T + TT - 1) / TT)), dim3(1024), 0, s, T, dPW1, dW, dB, (int8_t *)dQ,
                           ldq, dScales);
    };
    if (tt == 1) go(p2k::glu_dwconv_silu_quant<1>, 1);
    else if (tt == 4) go(p2k::glu_dwconv_silu_quant<4>, 4);
    else if (tt == 8) go(p2k::glu_dwconv_silu_quant<8>, 8);
    else go(p2k::glu_dwconv_silu_quant<2>, 2);   /* 2, the measured best, for any other value */
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

int p2h_silu(size_t n, float *dX, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (n == 0) return P2H_OK;
    if (!dX) return fail(P2H_E_ARG, "p2h_silu: null pointer");
    hipLaunchKernelGGL(p2k::silu_flat, dim3(blocks_of(n)), dim3(256), 0, stream_of(stream), n, dX);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

int p2h_add_residual(int T, float *dX, const float *dY, float alpha, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (T < 0) return fail(P2H_E_ARG, "p2h_add_residual: T = %d", T);
    if (T == 0) return P2H_OK;
    if (!dX || !dY) return fail(P2H_E_ARG, "p2h_add_residual: null pointer");
    const size_t n = (size_t)T * p2k::kD;
    hipLaunchKernelGGL(p2k::axpy_rows, dim3(blocks_of(n)), dim3(256), 0, stream_of(stream), n, alpha, dY, dX);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

/* ── GEMMs ──────────────────────────────────────────────────────────────────────────────────────────────────── */

int p2h_scale_c(int M, int N, float beta, float *dC, int ldc, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (M < 0 || N < 0 || (M > 0 && N > 0 && (!dC || ldc < N))) return fail(P2H_E_ARG, "p2h_scale_c: bad shape");
    if (beta == 1.0f || M == 0 || N == 0) return P2H_OK;
    size_t total = (size_t)M * N;
    hipLaunchKernelGGL(p2k::scale_c, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream_of(stream), M, N,
                       beta, dC, ldc);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

static int check_q(const char *who, int M, int K, const signed char *dQ, int ldq, const float *dScales)
{
    if (M < 0 || K < 0 || K % 4 != 0) return fail(P2H_E_ARG, "%s: K = %d must be a multiple of 4", who, K);
    if (M > 0 && (!dQ || !dScales)) return fail(P2H_E_ARG, "%s: NULL activations", who);
    if (M > 0 && (ldq < p2h_q_ld(K) || ldq % P2H_Q_KALIGN != 0 || !aligned(dQ, 16)))
        return fail(P2H_E_ARG, "%s: ldq = %d must be >= %d and a multiple of %d, Q 16-byte aligned", who, ldq,
                    p2h_q_ld(K), P2H_Q_KALIGN);
    return P2H_OK;
}

/* ── the int8 GEMM: plan and launch ──────────────────────────────────────────────────────────────────────────── */

}  // extern "C"

namespace {

/* Five-value tiles (gemm_fv): FM 16-row groups × FN 16-column groups per wave, 4 waves side by side along N, an LDS
 * ring of 4 stages of 128 K rows. */
using FvT = p2k::FvGeo<2, 1, 4, 4>;   /*  32 ×  64 */
using FvS = p2k::FvGeo<4, 1, 4, 4>;   /*  64 ×  64 */
using FvM = p2k::FvGeo<4, 2, 4, 4>;   /*  64 × 128 */
using FvL = p2k::FvGeo<8, 2, 4, 4>;   /* 128 × 128 */
using FvX = p2k::FvGeo<8, 4, 4, 4>;   /* 128 × 256 (int8w only: the two-plane mode would need twice the accumulators) */
using FvT8 = p2k::FvGeo<2, 1, 4, 8>;  /*  32 ×  64, 8 stages in flight */
using FvS8 = p2k::FvGeo<4, 1, 4, 8>;  /*  64 ×  64, 8 stages in flight */
using FvT6 = p2k::FvGeo<2, 1, 4, 6>;  /*  32 ×  64, 6 stages in flight */
/* Large-M tiles (int8w): two workgroups per CU, 4-bit selector records, outputs staged through LDS */
using FvW6 = p2k::FvGeo<6, 4, 4, 2>;  /*  96 × 256, 2 stages: K <= 1024 */
using FvWK = p2k::FvGeo<6, 2, 4, 2>;  /*  96 × 128, 2 stages: K > 1024, unsplit (504 tiles at M = 6000, N = 1024) */
/* Small-M tiles (gemm_fvs): operands straight to registers, K split across the four waves, 4-bit records */
using SmS = p2k::SmGeo<2, 2>;         /*  32 ×  32 */
using SmW = p2k::SmGeo<3, 4>;         /*  48 ×  64 (int8w) */
using SmD = p2k::SmGeo<2, 4, 2, 8>;   /*  32 ×  64, eight waves of four units each, all in flight: K > 1024 (int8w) */
/* Eight waves, one 128-row unit per load batch (int8w), for K > 1024: each wave's segment is four units, loaded one
 * unit ahead of the MFMAs, and a wave holds a quarter of the operand registers of SmS/SmD's two-unit batches */
using SmS8 = p2k::SmGeo<2, 2, 1, 8>;     /* 32 × 32 */
using SmW8 = p2k::SmGeo<3, 2, 1, 8>;     /* 48 × 32 */
/* Sixteen-row tiles (int8w) for a few dozen rows: a workgroup reads 16 activation rows instead of 32 or 48, so at
 * these M the tiles spread the rows and the weight columns over up to three times as many CUs, each reading less */
using SmQ = p2k::SmGeo<1, 1>;             /* 16 × 16, four waves (K <= 1024) */
using SmQ8 = p2k::SmGeo<1, 1, 4, 8>;      /* 16 × 16, eight waves (K > 1024), a segment's four units in one batch */
using SmR8 = p2k::SmGeo<1, 2, 1, 8>;      /* 16 × 32, eight waves (K > 1024) */
enum { FV_T = 0, FV_S = 1, FV_M = 2, FV_L = 3, FV_X = 4, FV_T8 = 5, FV_S8 = 6, FV_T6 = 7, FV_W6 = 8, FV_WK = 9,
       FV_SS = 10, FV_SW = 11, FV_SD = 12, FV_SS8 = 13, FV_SW8 = 14, FV_SQ = 15, FV_SQ8 = 16, FV_SR8 = 17,
       FV_COUNT = 18 };
/* calls f(G{}) with the small-M geometry of an int8w-only configuration; false for any other configuration */
template <class F>
bool with_small_geo(int cfg, F &&f)
{
    switch (cfg) {
    case FV_SW: f(SmW{}); return true;
    case FV_SD: f(SmD{}); return true;
    case FV_SS8: f(SmS8{}); return true;
    case FV_SW8: f(SmW8{}); return true;
    case FV_SQ: f(SmQ{}); return true;
    case FV_SQ8: f(SmQ8{}); return true;
    case FV_SR8: f(SmR8{}); return true;
    default: return false;
    }
}
const int kFvBM[FV_COUNT] = {FvT::BM, FvS::BM, FvM::BM, FvL::BM, FvX::BM, FvT8::BM, FvS8::BM, FvT6::BM, FvW6::BM,
                             FvWK::BM, SmS::BM, SmW::BM, SmD::BM, SmS8::BM, SmW8::BM, SmQ::BM, SmQ8::BM, SmR8::BM};
const int kFvBN[FV_COUNT] = {FvT::BN, FvS::BN, FvM::BN, FvL::BN, FvX::BN, FvT8::BN, FvS8::BN, FvT6::BN, FvW6::BN,
                             FvWK::BN, SmS::BN, SmW::BN, SmD::BN, SmS8::BN, SmW8::BN, SmQ::BN, SmQ8::BN, SmR8::BN};
/* gemm_fvs splits K among the waves of a workgroup, one 1024-row fold block at most per segment, so K <= 4096 */
inline bool small_ok(int K) { return K <= 4 * p2k::kFoldRows; }
inline bool is_small(int cfg) { return cfg >= FV_SS && cfg < FV_COUNT; }
/* the small tiles that exist for int8w only (the two-plane mode runs SmS in their place) */
inline bool int8w_only(int cfg) { return cfg > FV_SS && cfg < FV_COUNT; }

/* int8-table tiles (gemm_i8): activation rows × table columns, waves (m × n), K rows per LDS stage */
using G64 = p2k::Geo<64, 64, 2, 2, 256>;
using G128 = p2k::Geo<128, 128, 2, 2, 128>;
using G3264 = p2k::Geo<32, 64, 2, 2, 256>;   /* int8-table GEMMs: K <= 1024 when 64 x 64 tiles leave CUs idle */

struct Plan {
    int cfg, splits, split_rows, tiles_m, tiles_n;
    size_t part_bytes;
};

/* Tile and K split of a five-value call. A split is a whole number of 128-row units inside one 1024-row fold block;
 * it runs only with a workspace, for K > 1024 (its int32 partials cost splits × M × N × 4 bytes of traffic, worth
 * it only where the output is small next to K). P2H_TILE and P2H_SPLIT_ROWS (−1: never) override the choice. */
Plan make_plan(int mode, int M, int N, int K, bool can_split)
{
    Plan p;
    int cfg;
    if (M <= 1024) {
        /* Small M: the register-streaming kernel (gemm_fvs). Measured on MI355X with the weights from HBM:
         *  - sixteen-row tiles while they fit the CUs in one round (K > 1024: eight waves, 16 × 16, then 16 × 32;
         *    K <= 1024: four waves, two workgroups per CU): a workgroup then reads 16 activation rows instead of 32
         *    or 48 (M = 38, 4096 -> 1024: 4.28 against 5.13 µs; 1024 -> 1024: 2.96 against 3.36 µs);
         *  - K > 1024: eight waves of one unit per batch while their tiles fit in one round, 32 × 32 up to 256 rows
         *    (14 % faster at M = 250), 48 × 32 up to 384 (6 % at M = 375); then the eight-wave 32 × 64, whose
         *    segments' loads are all in flight, where those tiles fill between half and all of the CUs;
         *  - K <= 1024: 48 × 64 for wide outputs at a few hundred rows (N >= 3072, M >= 256; 32 × 32 wins up to
         *    N = 2048), else 32 × 32.
         * Beyond a thousand rows: the two-workgroups-per-CU tiles on 4-bit records (int8w) or 128 × 128 (the
         * two-plane mode needs twice the accumulators). */
        const int cus_ = g_cus > 0 ? g_cus : 256;
        auto tiles_of = [&](int bm, int bn) { return (long long)((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
        const long long sd_tiles = tiles_of(SmD::BM, SmD::BN);
        const bool deep = K > p2k::kFoldRows && mode == P2H_INT8W;
        const bool w8 = mode == P2H_INT8W;
        cfg = !small_ok(K) ? FV_T
              : (deep && tiles_of(16, 16) <= cus_) ? FV_SQ8
              : (deep && tiles_of(16, 32) <= cus_) ? FV_SR8
              : (w8 && !deep && tiles_of(16, 16) <= 2 * cus_) ? FV_SQ
              : (K <= p2k::kFoldRows && N >= 3072 && M >= 256) ? FV_SW
              : (deep && tiles_of(SmS8::BM, SmS8::BN) <= cus_) ? FV_SS8
              : (deep && tiles_of(SmW8::BM, SmW8::BN) <= cus_) ? FV_SW8
              : (deep && 2 * sd_tiles >= cus_ && sd_tiles <= cus_) ? FV_SD
              : FV_SS;
    }
    else {
        /* int8w: 96 × 256 for K <= 1024 unless its tiles leave every CU one workgroup at most (a lone workgroup's K
         * loop is no faster than a pair's), then 96 × 128, twice the workgroups: 1024 → 1024 at M = 6000 11.2–11.6
         * against 12.3 µs, at M = 3000 7.8 against 11.0; 1024 → 4096 at M = 1500 10.8 against 12.1; 1024 → 3072 at
         * M = 2000 11.0 against 12.2. With more tiles than CUs 96 × 256 wins or ties (M = 4099: 26.6 against 27.8 µs;
         * 1024 → 2048 at M = 6000: 19.3 against 21.4; 1024 → 3072 at M = 4000: 18.7 against 20.6). */
        const int cus_ = g_cus > 0 ? g_cus : 256;
        const long long w6_tiles = (long long)((M + 95) / 96) * ((N + 255) / 256);
        cfg = mode == P2H_INT8W ? (K > p2k::kFoldRows || w6_tiles <= cus_ ? FV_WK : FV_W6) : FV_L;
    }
    if (switch_of(g_sw.tile) != kUnset) cfg = switch_of(g_sw.tile);
    if (cfg < 0 || cfg >= FV_COUNT) cfg = FV_S;
    if (mode == P2H_INT8 && (cfg == FV_X || cfg == FV_W6 || cfg == FV_WK)) cfg = FV_L;
    if (mode == P2H_INT8 && int8w_only(cfg)) cfg = FV_SS;
    if (is_small(cfg) && !small_ok(K)) cfg = FV_T;
    /* these never split K across workgroups: the fold stays in the kernel */
    const bool large = cfg == FV_W6 || cfg == FV_WK || is_small(cfg);
    p.cfg = cfg;
    p.tiles_m = (M + kFvBM[cfg] - 1) / kFvBM[cfg];
    p.tiles_n = (N + kFvBN[cfg] - 1) / kFvBN[cfg];
    const int tiles = p.tiles_m * p.tiles_n;
    const int cus = g_cus > 0 ? g_cus : 256;
    p.splits = 1;
    p.split_rows = K > 0 ? K : 1;
    int rows = 0;
    if (K > p2k::kFoldRows) rows = (M <= 64 && tiles * (K / 512) <= 2 * cus) ? 512 : p2k::kFoldRows;
    const int forced = switch_of(g_sw.split_rows);
    if (forced < 0) rows = 0;
    else if (forced > 0 && forced <= p2k::kFoldRows && p2k::kFoldRows % forced == 0 && forced % 128 == 0) rows = forced;
    if (can_split && !large && K > 0 && rows > 0 && (K + rows - 1) / rows > 1) {
        p.split_rows = rows;
        p.splits = (K + rows - 1) / rows;
    }
    const size_t planes = mode == P2H_INT8 ? 2 : 1;
    p.part_bytes = p.splits > 1 ? align_up(planes * p.splits * (size_t)M * N * 4, 256) : 0;
    return p;
}

/* Small-M tiles on a grid of XCD blocks (fvs_tile) where the weight records (K·N/2 bytes) weigh less than twice the
 * quantised rows (M·K): four rows of XCDs, each L2 then fetching a quarter of the rows and half of the records
 * instead of all the rows. Graph replays on MI355X: the M = 375 FFN pair 22.7 -> 21.5 us, the 216-linear sweep
 * 1942 -> 1917 us, the 24-block stack 3.19 -> 3.17 ms. Four rows of XCDs for every shape gave the pair 21.9 us and
 * the stack 3.21 ms; two rows, or one, were slower. Returns the rows of XCDs, or 0 for the plain order. */
int xcd_rows_of(const Plan &p, int M, int N)
{
    int a = switch_of(g_sw.xcd_rows);
    if (a < 0) a = (long long)N < 4LL * M ? -a : 0;   /* negative: only where N < 4·M */
    if ((a == 1 || a == 2 || a == 4 || a == 8) && is_small(p.cfg) && p.splits == 1 && p.tiles_m % a == 0 &&
        p.tiles_n % (8 / a) == 0)
        return a;
    return 0;
}

p2k::GemmArgs gemm_args(int M, int N, int K, float alpha, float beta, const signed char *dQ, int ldq,
                        const float *dScales, float *dC, int ldc, const Plan &p, void *split_ws)
{
    p2k::GemmArgs g;
    memset(&g, 0, sizeof g);
    g.M = M; g.N = N; g.K = K;
    g.alpha = alpha; g.beta = beta;
    g.Q = (const int8_t *)dQ; g.ldq = ldq; g.a_scales = dScales;
    g.kq = (int)align_up((size_t)K, P2H_Q_KALIGN);
    g.kst = ldq / 64;
    g.mg_last = (int)(align_up((size_t)M, 16) / 16) - 1;
    g.ng_last = N / 16 - 1;
    g.C = dC; g.ldc = ldc;
    g.c_vec4 = dC && (ldc % 4 == 0) && aligned(dC, 16);
    g.c_wt = switch_of(g_sw.dev_scope_stores) ? 1 : 0;
    g.tiles_n = p.tiles_n; g.tiles_m = p.tiles_m;
    g.splits = p.splits; g.split_rows = p.split_rows;
    g.xcd_rows = xcd_rows_of(p, M, N);
    if (p.splits > 1) g.part = (int32_t *)split_ws;
    return g;
}

/* the large-M tiles: unsplit, two workgroups per CU, 4-bit records (in registers, or through the LDS ring with the
 * activation rows), staged output rows */
template <class G>
void launch_fv_large(const p2k::GemmArgs &g, const Plan &p, hipStream_t s)
{
    const dim3 grid((unsigned)((size_t)p.tiles_m * p.tiles_n)), block(G::NT);
    if (switch_of(g_sw.records_in_regs)) {
        if (g.K > p2k::kFoldRows) hipLaunchKernelGGL((p2k::gemm_fv_rb<G, true>), grid, block, 0, s, g);
        else hipLaunchKernelGGL((p2k::gemm_fv_rb<G, false>), grid, block, 0, s, g);
        return;
    }
    if (g.K > p2k::kFoldRows)
        hipLaunchKernelGGL((p2k::gemm_fv<G, p2k::MODE_INT8W, p2k::OUT_F32, true, false, 2, true>), grid, block, 0,
                           s, g);
    else
        hipLaunchKernelGGL((p2k::gemm_fv<G, p2k::MODE_INT8W, p2k::OUT_F32, false, false, 2, true>), grid, block,
                           0, s, g);
}

template <class G, int MODE>
void launch_fv(const p2k::GemmArgs &g, const Plan &p, hipStream_t s)
{
    const dim3 grid((unsigned)((size_t)p.tiles_m * p.tiles_n * p.splits)), block(G::NT);
    if (p.splits > 1) {
        hipLaunchKernelGGL((p2k::gemm_fv<G, MODE, p2k::OUT_F32, false, true>), grid, block, 0, s, g);
        const size_t quads = (size_t)g.M * (g.N / 4);
        hipLaunchKernelGGL((p2k::fold_splits<MODE == p2k::MODE_INT8>), dim3((unsigned)((quads + 255) / 256)),
                           dim3(256), 0, s, g);
    } else if (g.K > p2k::kFoldRows) {
        hipLaunchKernelGGL((p2k::gemm_fv<G, MODE, p2k::OUT_F32, true, false>), grid, block, 0, s, g);
    } else {
        hipLaunchKernelGGL((p2k::gemm_fv<G, MODE, p2k::OUT_F32, false, false>), grid, block, 0, s, g);
    }
}

template <class G, int MODE>
void launch_fvs(const p2k::GemmArgs &g, const Plan &p, hipStream_t s)
{
    hipLaunchKernelGGL((p2k::gemm_fvs<G, MODE>), dim3((unsigned)((size_t)p.tiles_m * p.tiles_n)), dim3(G::NT), 0, s,
                       g);
}

template <int MODE>
void launch_fv_cfg(const p2k::GemmArgs &g, const Plan &p, hipStream_t s)
{
    switch (p.cfg) {
    case FV_SS: launch_fvs<SmS, MODE>(g, p, s); break;
    case FV_SW: case FV_SD: case FV_SS8: case FV_SW8: case FV_SQ: case FV_SQ8: case FV_SR8:
        if (MODE != p2k::MODE_INT8W) { launch_fvs<SmS, MODE>(g, p, s); break; }   /* make_plan maps int8 away */
        with_small_geo(p.cfg, [&](auto geo) { launch_fvs<decltype(geo), p2k::MODE_INT8W>(g, p, s); });
        break;
    case FV_T: launch_fv<FvT, MODE>(g, p, s); break;
    case FV_S: launch_fv<FvS, MODE>(g, p, s); break;
    case FV_M: launch_fv<FvM, MODE>(g, p, s); break;
    case FV_T8: launch_fv<FvT8, MODE>(g, p, s); break;
    case FV_S8: launch_fv<FvS8, MODE>(g, p, s); break;
    case FV_T6: launch_fv<FvT6, MODE>(g, p, s); break;
    case FV_W6: if (MODE == p2k::MODE_INT8W) { launch_fv_large<FvW6>(g, p, s); break; } /* fall through */
    case FV_WK: if (MODE == p2k::MODE_INT8W) { launch_fv_large<FvWK>(g, p, s); break; } /* fall through */
    case FV_X: if (MODE == p2k::MODE_INT8W) { launch_fv<FvX, p2k::MODE_INT8W>(g, p, s); break; } /* fall through */
    default: launch_fv<FvL, MODE>(g, p, s); break;
    }
}

int check_split_ws(const char *who, const Plan &p, void *ws, size_t ws_bytes)
{
    if (p.splits <= 1) return P2H_OK;
    if (!ws || ws_bytes < p.part_bytes || !aligned(ws, 256))
        return fail(P2H_E_WORKSPACE, "%s: split workspace of %zu bytes needed", who, p.part_bytes);
    return P2H_OK;
}

}  // namespace

extern "C" {

const char *p2h_fvb_plan(int mode, int M, int N, int K, int with_workspace)
{
    static thread_local char buf[160];
    if (ensure_init() || M <= 0 || N <= 0 || K <= 0) return "";
    Plan p = make_plan(mode == P2H_INT8 ? P2H_INT8 : P2H_INT8W, M, N, K, with_workspace != 0);
    if (is_small(p.cfg)) {
        const int a = xcd_rows_of(p, M, N);
        char grid[32] = "";
        if (a > 0) snprintf(grid, sizeof grid, ", XCD grid %dx%d", a, 8 / a);
        snprintf(buf, sizeof buf, "tile %dx%d, K split across the workgroup's waves, fold in LDS%s", kFvBM[p.cfg],
                 kFvBN[p.cfg], grid);
    }
    else
        snprintf(buf, sizeof buf, "tile %dx%d, %d split%s of %d rows%s%s", kFvBM[p.cfg], kFvBN[p.cfg], p.splits,
                 p.splits > 1 ? "s" : "", p.split_rows,
                 p.splits > 1 ? " + fold" : (K > p2k::kFoldRows ? ", folds in registers" : ""),
                 (p.cfg == FV_W6 || p.cfg == FV_WK) && mode != P2H_INT8 && switch_of(g_sw.records_in_regs)
                     ? ", weight records in registers" : "");
    return buf;
}

size_t p2h_fvb_q8a_workspace_bytes(int mode, int M, int N, int K)
{
    if (ensure_init() || M <= 0 || N <= 0 || K <= 0 || (mode != P2H_INT8W && mode != P2H_INT8)) return 0;
    Plan p = make_plan(mode, M, N, K, true);
    return p.part_bytes;   /* the split partials, or 0 when the call would not split */
}

static int fvb_gemm_q8a(int mode, int M, int N, int K, float alpha, const signed char *dQ, int ldq,
                        const float *dScales, const P2hWeight *w, float beta, float *dC, int ldc, void *workspace,
                        size_t workspace_bytes, const P2hWeight *next, void *stream, bool silu = false);

int p2h_fvb_gemm_q8a(int mode, int M, int N, int K, float alpha, const signed char *dQ, int ldq,
                     const float *dScales, const P2hWeight *w, float beta, float *dC, int ldc, void *workspace,
                     size_t workspace_bytes, void *stream)
{
    return fvb_gemm_q8a(mode, M, N, K, alpha, dQ, ldq, dScales, w, beta, dC, ldc, workspace, workspace_bytes,
                        nullptr, stream);
}

int p2h_fvb_gemm_q8a_next(int mode, int M, int N, int K, float alpha, const signed char *dQ, int ldq,
                          const float *dScales, const P2hWeight *w, float beta, float *dC, int ldc, void *workspace,
                          size_t workspace_bytes, const P2hWeight *next, void *stream)
{
    return fvb_gemm_q8a(mode, M, N, K, alpha, dQ, ldq, dScales, w, beta, dC, ldc, workspace, workspace_bytes, next,
                        stream);
}

int p2h_fvb_gemm_q8a_silu(int mode, int M, int N, int K, float alpha, const signed char *dQ, int ldq,
                          const float *dScales, const P2hWeight *w, float *dC, void *workspace,
                          size_t workspace_bytes, void *stream)
{
    return fvb_gemm_q8a(mode, M, N, K, alpha, dQ, ldq, dScales, w, 0.0f, dC, N, workspace, workspace_bytes, nullptr,
                        stream, true);
}

/* silu: C = silu_p2(alpha·A·W) with beta 0, ldc = N and N % 8 == 0 (p2_swish over whole rows: every element in
 * the eight-wide body); small-M tiles apply it in their epilogue, the others by p2h_silu after the GEMM. */
static int fvb_gemm_q8a(int mode, int M, int N, int K, float alpha, const signed char *dQ, int ldq,
                        const float *dScales, const P2hWeight *w, float beta, float *dC, int ldc, void *workspace,
                        size_t workspace_bytes, const P2hWeight *next, void *stream, bool silu)
{
    if (int rc = ensure_init()) return rc;
    if (silu && (beta != 0.0f || ldc != N || N % 8 != 0))
        return fail(P2H_E_ARG, "p2h_fvb_gemm_q8a_silu: needs beta 0, ldc = N and N %% 8 == 0 (N = %d)", N);
    if (mode != P2H_INT8W && mode != P2H_INT8)
        return fail(P2H_E_ARG, "p2h_fvb_gemm_q8a: mode %d is not an int8 mode", mode);
    if (!w || w->N != N || w->K != K)
        return fail(P2H_E_ARG, "p2h_fvb_gemm_q8a: weight is [%d, %d], call asks [%d, %d]", w ? w->K : -1,
                    w ? w->N : -1, K, N);
    if (int rc = check_q("p2h_fvb_gemm_q8a", M, K, dQ, ldq, dScales)) return rc;
    if (M > 0 && (!dC || ldc < N)) return fail(P2H_E_ARG, "p2h_fvb_gemm_q8a: C or ldc invalid");
    hipStream_t s = stream_of(stream);
    if (M == 0) return P2H_OK;
    if (alpha == 0.0f) return p2h_scale_c(M, N, beta, dC, ldc, s);            /* blas.c:1434 */
    if (K == 0)   /* no K block runs (SiLU of the zero product: zeros) */
        return (beta != 0.0f || silu) ? p2h_scale_c(M, N, beta, dC, ldc, s) : P2H_OK;
    Plan p = make_plan(mode, M, N, K, workspace != nullptr);
    if (int rc = check_split_ws("p2h_fvb_gemm_q8a", p, workspace, workspace_bytes)) return rc;
    p2k::GemmArgs g = gemm_args(M, N, K, alpha, beta, dQ, ldq, dScales, dC, ldc, p, workspace);
    g.rec = w->rec4;
    g.units = w->units; g.clo = w->clo;
    if (next && is_small(p.cfg)) {   /* the records the next call reads */
        const size_t bytes = (size_t)(next->N / 16) * next->units * 1024;
        g.warm = next->rec4;
        g.warm_lines = (int)std::min<size_t>((bytes + 127) / 128, 0x7fffffff);
    }
    const bool silu_here = silu && is_small(p.cfg);
    g.act = silu_here ? 1 : 0;
    if (mode == P2H_INT8W) {
        g.c1 = w->hi; g.c1_hi = 1;
        launch_fv_cfg<p2k::MODE_INT8W>(g, p, s);
    } else {
        g.c1 = w->lo; g.c2 = w->hi;
        launch_fv_cfg<p2k::MODE_INT8>(g, p, s);
    }
    HIPCHK(hipGetLastError());
    if (silu && !silu_here) return p2h_silu((size_t)M * N, dC, s);
    return P2H_OK;
}

int p2h_fvb_gemm_q8a_grouped(int mode, int M, int N, int K, float alpha, const signed char *dQ, int ldq,
                             const float *dScales, const P2hWeight *const *w, int groups, float beta,
                             float *const *dC, int ldc, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (mode != P2H_INT8W && mode != P2H_INT8)
        return fail(P2H_E_ARG, "p2h_fvb_gemm_q8a_grouped: mode %d is not an int8 mode", mode);
    if (groups < 0 || groups > p2k::kMaxGroups || (groups > 0 && (!w || !dC)))
        return fail(P2H_E_ARG, "p2h_fvb_gemm_q8a_grouped: %d groups (at most %d, non-NULL arrays)", groups,
                    p2k::kMaxGroups);
    for (int q = 0; q < groups; q++) {
        if (!w[q] || w[q]->N != N || w[q]->K != K)
            return fail(P2H_E_ARG, "p2h_fvb_gemm_q8a_grouped: weight %d is not [%d, %d]", q, K, N);
        if (M > 0 && (!dC[q] || ldc < N)) return fail(P2H_E_ARG, "p2h_fvb_gemm_q8a_grouped: C %d or ldc invalid", q);
    }
    if (int rc = check_q("p2h_fvb_gemm_q8a_grouped", M, K, dQ, ldq, dScales)) return rc;
    hipStream_t s = stream_of(stream);
    if (M == 0 || groups == 0) return P2H_OK;
    Plan p = make_plan(mode, M, N, K, false);
    /* the launch covers groups · N columns of the same rows: its tile follows the single-call rule at that width
     * (measured, 24 weights of 1024 × 1024 at M = 749: 56.5 µs with 48 × 64 tiles against 63 µs with 32 × 32) */
    bool wide = false;   /* the large-M kernel's 96 × 256 tiles, where they number at least one per CU */
    if (is_small(p.cfg) && mode == P2H_INT8W &&
        make_plan(mode, M, (int)std::min<long long>((long long)N * groups, 1 << 30), K, false).cfg == FV_SW) {
        const long long w6_tiles = (long long)((M + FvW6::BM - 1) / FvW6::BM) * ((N + FvW6::BN - 1) / FvW6::BN) * groups;
        const int forced_tile = switch_of(g_sw.tile);
        wide = M >= 512 && w6_tiles >= (g_cus > 0 ? g_cus : 256) && (forced_tile == kUnset || forced_tile < 0);
        p.cfg = wide ? FV_W6 : FV_SW;
        p.tiles_m = wide ? (M + FvW6::BM - 1) / FvW6::BM : (M + SmW::BM - 1) / SmW::BM;
        p.tiles_n = wide ? (N + FvW6::BN - 1) / FvW6::BN : (N + SmW::BN - 1) / SmW::BN;
    }
    if (alpha == 0.0f || K == 0 || (!is_small(p.cfg) && !wide)) {   /* one call per weight: the same kernels, unsplit */
        for (int q = 0; q < groups; q++)
            if (int rc = p2h_fvb_gemm_q8a(mode, M, N, K, alpha, dQ, ldq, dScales, w[q], beta, dC[q], ldc, nullptr, 0,
                                          stream))
                return rc;
        return P2H_OK;
    }
    if (beta != 0.0f && beta != 1.0f) {   /* pre-scale, as the single entry does (blas.c:1436) */
        for (int q = 0; q < groups; q++)
            if (int rc = p2h_scale_c(M, N, beta, dC[q], ldc, s)) return rc;
        beta = 1.0f;
    }
    p2k::GemmArgs g = gemm_args(M, N, K, alpha, beta, dQ, ldq, dScales, dC[0], ldc, p, nullptr);
    p2k::GroupArgs ga;
    memset(&ga, 0, sizeof ga);
    for (int q = 0; q < groups; q++) {
        ga.rec[q] = w[q]->rec4; ga.clo[q] = w[q]->clo; ga.C[q] = dC[q];
        ga.c1[q] = mode == P2H_INT8W ? w[q]->hi : w[q]->lo;
        ga.c2[q] = w[q]->hi;
        if (!aligned(dC[q], 16)) g.c_vec4 = 0;
    }
    g.units = w[0]->units;
    g.c1_hi = mode == P2H_INT8W ? 1 : 0;
    /* the kernel of the plan's tile: the grid and g.tiles_n/tiles_m were sized for exactly that tile */
    const dim3 grid((unsigned)((size_t)p.tiles_m * p.tiles_n), (unsigned)groups);
    if (wide)
        hipLaunchKernelGGL((p2k::gemm_fv_grouped<FvW6, false>), grid, dim3(FvW6::NT), 0, s, g, ga);
    else if (mode == P2H_INT8)   /* make_plan gives the two-plane mode 32 x 32 tiles only */
        hipLaunchKernelGGL((p2k::gemm_fvs_grouped<SmS, p2k::MODE_INT8>), grid, dim3(SmS::NT), 0, s, g, ga);
    else if (p.cfg == FV_SS)
        hipLaunchKernelGGL((p2k::gemm_fvs_grouped<SmS, p2k::MODE_INT8W>), grid, dim3(SmS::NT), 0, s, g, ga);
    else if (!with_small_geo(p.cfg, [&](auto geo) {
                 using G = decltype(geo);
                 hipLaunchKernelGGL((p2k::gemm_fvs_grouped<G, p2k::MODE_INT8W>), grid, dim3(G::NT), 0, s, g, ga);
             }))
        return fail(P2H_E_ARG, "p2h_fvb_gemm_q8a_grouped: no grouped kernel for tile %d", p.cfg);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

int p2h_fvb_acc_i32(int mode, int M, int N, int K, const signed char *dQ, int ldq, const P2hWeight *w,
                    int32_t *dAcc, int32_t *dAcc2, int ldacc, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (mode != P2H_INT8W && mode != P2H_INT8) return fail(P2H_E_ARG, "p2h_fvb_acc_i32: mode %d", mode);
    if (!w || w->N != N || w->K != K) return fail(P2H_E_ARG, "p2h_fvb_acc_i32: weight shape mismatch");
    if (M > 0 && !dQ) return fail(P2H_E_ARG, "p2h_fvb_acc_i32: NULL activations");
    if (int rc = check_q("p2h_fvb_acc_i32", M, K, dQ, ldq, (const float *)dAcc)) return rc;
    if (M > 0 && (!dAcc || ldacc < N || ldacc % 4 != 0 || !aligned(dAcc, 16) ||
                  (mode == P2H_INT8 && (!dAcc2 || !aligned(dAcc2, 16)))))
        return fail(P2H_E_ARG, "p2h_fvb_acc_i32: accumulators must be 16-byte aligned with ldacc %% 4 == 0");
    if (M == 0) return P2H_OK;
    Plan p = make_plan(mode, M, N, K, false);
    p.cfg = FV_L;
    p.splits = 1;
    p.split_rows = K;
    p.tiles_m = (M + FvL::BM - 1) / FvL::BM;
    p.tiles_n = (N + FvL::BN - 1) / FvL::BN;
    p2k::GemmArgs g = gemm_args(M, N, K, 1.0f, 0.0f, dQ, ldq, nullptr, nullptr, 0, p, nullptr);
    g.rec = w->rec4; g.units = w->units; g.clo = w->clo;
    g.acc1 = dAcc; g.acc2 = dAcc2; g.ldacc = ldacc;
    hipStream_t s = stream_of(stream);
    const dim3 grid((unsigned)((size_t)p.tiles_m * p.tiles_n)), block(FvL::NT);
    if (mode == P2H_INT8W)
        hipLaunchKernelGGL((p2k::gemm_fv<FvL, p2k::MODE_INT8W, p2k::OUT_ACC, false, false>), grid, block, 0,
                           s, g);
    else
        hipLaunchKernelGGL((p2k::gemm_fv<FvL, p2k::MODE_INT8, p2k::OUT_ACC, false, false>), grid, block, 0, s,
                           g);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

static int launch_exact(int bkind, const p2k::ExactArgs &g0, hipStream_t s)
{
    p2k::ExactArgs g = g0;
    g.tiles_n = (g.N + p2k::EBN - 1) / p2k::EBN;
    size_t tiles = (size_t)g.tiles_n * ((g.M + p2k::EBM - 1) / p2k::EBM);
    if (tiles == 0) return P2H_OK;
    if (bkind == p2k::EXB_FV)
        hipLaunchKernelGGL(p2k::gemm_exact<p2k::EXB_FV>, dim3((unsigned)tiles), dim3(256), 0, s, g);
    else
        hipLaunchKernelGGL(p2k::gemm_exact<p2k::EXB_Q8>, dim3((unsigned)tiles), dim3(256), 0, s, g);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

/* The exact five-value route on the fp32 matrix cores (gemm_xf): 32 × 64 tiles, or 32 × 32 where 32 × 64 would leave
 * fewer than two workgroups per CU; rows staged through LDS by direct loads where K % 128 == 0 and the rows allow
 * 16-byte loads (the same bits as the register path, which P2H_XF_STAGED=0 selects). P2H_EXACT_CHAIN=1 selects
 * gemm_exact instead, the reference's per-output fmaf chain bit for bit; P2H_XF_TILE = 32 or 64 forces the tile
 * width. */
}  // extern "C"

namespace {

template <int FM, int FN>
void launch_xf_tile(const p2k::ExactArgs &g, hipStream_t s)
{
    const dim3 grid((unsigned)((size_t)g.tiles_n * ((g.M + 16 * FM - 1) / (16 * FM)))), block(256);
    const bool vec = g.K % 4 == 0 && g.lda % 4 == 0 && aligned(g.A, 16);
    const bool staged = vec && g.K % 128 == 0 && switch_of(g_sw.xf_staged) != 0;
    if (staged) hipLaunchKernelGGL((p2k::gemm_xf<FM, FN, true, true>), grid, block, 0, s, g);
    else if (vec) hipLaunchKernelGGL((p2k::gemm_xf<FM, FN, true>), grid, block, 0, s, g);
    else hipLaunchKernelGGL((p2k::gemm_xf<FM, FN, false>), grid, block, 0, s, g);
}

int launch_xf(const p2k::ExactArgs &g0, hipStream_t s)
{
    p2k::ExactArgs g = g0;
    const long long cus = g_cus > 0 ? g_cus : 256;
    /* measured at M = 38 to 749 (the weights from HBM, the same bits for every tile): 16 × 16 tiles while they
     * number at most six per CU (M = 38, 4096 -> 1024: 13.3 against 27.2 µs; M = 375, 4096 -> 1024: 41.4 against
     * 44.9 µs), then 32 × 64 where those fill three workgroups per CU, else 32 × 32 (M = 375, 1024 -> 3072: 29.6
     * against 33.3 µs for 32 × 64) */
    const long long t16 = (long long)((g.N + 15) / 16) * ((g.M + 15) / 16);
    const long long t64 = (long long)((g.N + 63) / 64) * ((g.M + 31) / 32);
    int bm = t16 <= 6 * cus ? 16 : 32;
    int bn = bm == 16 ? 16 : (t64 >= 3 * cus ? 64 : 32);
    const int forced = switch_of(g_sw.xf_tile);
    if (forced == 32 || forced == 64) { bm = 32; bn = forced; }
    if (forced == 1616 || forced == 1632 || forced == 1664) { bm = 16; bn = forced - 1600; }
    g.tiles_n = (g.N + bn - 1) / bn;
    if (bm == 16 && bn == 16) launch_xf_tile<1, 1>(g, s);
    else if (bm == 16 && bn == 32) launch_xf_tile<1, 2>(g, s);
    else if (bm == 16) launch_xf_tile<1, 4>(g, s);
    else if (bn == 64) launch_xf_tile<2, 4>(g, s);
    else launch_xf_tile<2, 2>(g, s);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

}  // namespace

extern "C" {

static size_t quant_area(int M, int K) { return align_up(p2h_q_bytes(M, K), 256) + align_up((size_t)M * 4, 256); }

/* Workspace of the fp32-input entries: [split partials][quantised rows][row scales]. */
size_t p2h_fvb_workspace_bytes(int mode, int M, int N, int K)
{
    if (ensure_init() || mode == P2H_EXACT || M <= 0 || N <= 0 || K <= 0 || K % 4 != 0) return 0;
    Plan p = make_plan(mode == P2H_INT8 ? P2H_INT8 : P2H_INT8W, M, N, K, true);
    return p.part_bytes + quant_area(M, K);
}

static int quant_into_workspace(const char *who, int mode, int M, int N, int K, const float *dA, int lda,
                                void *workspace, size_t workspace_bytes, signed char **dQ, float **dS,
                                hipStream_t s)
{
    size_t need = p2h_fvb_workspace_bytes(mode, M, N, K);
    if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
        return fail(P2H_E_WORKSPACE, "%s: workspace of %zu bytes (256-byte aligned) needed, %zu given", who, need,
                    workspace_bytes);
    *dQ = (signed char *)workspace + (need - quant_area(M, K));
    *dS = (float *)((char *)*dQ + align_up(p2h_q_bytes(M, K), 256));
    return p2h_quant_rows(M, K, dA, lda, *dQ, p2h_q_ld(K), *dS, s);
}

/* The exact route after p2h_fvb_gemm's checks (M > 0). silu: the block's feed-forward up-projection, h =
 * p2_swish(A·W) (encoder.c:353-354) with the SiLU in the matrix-core GEMM's epilogue; beta 0, ldc = N and N % 8 == 0,
 * where p2_swish's eight-wide body (silu_p2) covers every element, so the bits are those of the GEMM followed by
 * p2h_silu. The fmaf-chain route keeps the separate pass. */
static int exact_gemm(int M, int N, int K, float alpha, const float *dA, int lda, const P2hWeight *w, float beta,
                      float *dC, int ldc, hipStream_t s, bool silu)
{
    if (silu && (beta != 0.0f || ldc != N || N % 8 != 0))
        return fail(P2H_E_ARG, "exact GEMM with SiLU: needs beta 0, ldc = N and N %% 8 == 0");
    p2k::ExactArgs g;
    memset(&g, 0, sizeof g);
    g.M = M; g.N = N; g.K = K; g.alpha = alpha; g.beta = beta;
    g.A = dA; g.lda = lda;
    g.lo = w->lo; g.hi = w->hi;
    g.C = dC; g.ldc = ldc;
    g.rec = w->rec4; g.units = w->units;
    if (switch_of(g_sw.exact_chain) != 0 || K == 0) {
        if (int rc = launch_exact(p2k::EXB_FV, g, s)) return rc;
        return silu ? p2h_silu((size_t)M * N, dC, s) : P2H_OK;
    }
    g.act = silu ? 1 : 0;
    return launch_xf(g, s);
}

int p2h_fvb_gemm(int mode, int M, int N, int K, float alpha, const float *dA, int lda, const P2hWeight *w,
                 float beta, float *dC, int ldc, void *workspace, size_t workspace_bytes, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (mode != P2H_INT8W && mode != P2H_INT8 && mode != P2H_EXACT)
        return fail(P2H_E_ARG, "p2h_fvb_gemm: unknown mode %d", mode);
    if (!w || w->N != N || w->K != K)
        return fail(P2H_E_ARG, "p2h_fvb_gemm: weight is [%d, %d], call asks [%d, %d]", w ? w->K : -1,
                    w ? w->N : -1, K, N);
    if (M < 0 || K < 0) return fail(P2H_E_ARG, "p2h_fvb_gemm: negative shape");
    if (M > 0 && (!dC || ldc < N || (K > 0 && (!dA || lda < K)))) return fail(P2H_E_ARG, "p2h_fvb_gemm: bad A/C");
    hipStream_t s = stream_of(stream);
    if (M == 0) return P2H_OK;
    if (alpha == 0.0f) return p2h_scale_c(M, N, beta, dC, ldc, s);   /* blas.c:1488 */
    if (mode != P2H_EXACT && K % 4 == 0) {                            /* blas.c:1490-1493 */
        if (beta != 0.0f && beta != 1.0f) {
            if (int rc = p2h_scale_c(M, N, beta, dC, ldc, s)) return rc;
            beta = 1.0f;
        }
        if (K == 0) return P2H_OK;
        signed char *dQ;
        float *dS;
        if (int rc = quant_into_workspace("p2h_fvb_gemm", mode, M, N, K, dA, lda, workspace, workspace_bytes, &dQ,
                                          &dS, s))
            return rc;
        return p2h_fvb_gemm_q8a(mode, M, N, K, alpha, dQ, p2h_q_ld(K), dS, w, beta, dC, ldc, workspace,
                                (size_t)((char *)dQ - (char *)workspace), s);
    }
    return exact_gemm(M, N, K, alpha, dA, lda, w, beta, dC, ldc, s, false);
}

size_t p2h_noalloc_scratch_bytes(void) { return kScratchBytes; }

int p2h_fvb_gemm_noalloc(int mode, int M, int N, int K, float alpha, const float *dA, int lda, const P2hWeight *w,
                         float beta, float *dC, int ldc, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (!stream)
        return fail(P2H_E_ARG, "p2h_fvb_gemm_noalloc: needs the caller's stream (this library's per-thread stream "
                               "is created on first use)");
    if (mode != P2H_INT8W && mode != P2H_INT8 && mode != P2H_EXACT)
        return fail(P2H_E_ARG, "p2h_fvb_gemm_noalloc: unknown mode %d", mode);
    const size_t need = p2h_fvb_workspace_bytes(mode, M, N, K);   /* 0 on the exact route */
    if (need > kScratchBytes)
        return fail(P2H_E_WORKSPACE,
                    "p2h_fvb_gemm_noalloc: %d x %d x %d needs %zu bytes of workspace, above the %zu-byte scratch "
                    "array; use p2h_fvb_gemm with a workspace",
                    M, K, N, need, kScratchBytes);
    void *ws = nullptr;
    if (need > 0)
        if (int rc = scratch_of_current_device(&ws)) return rc;
    return p2h_fvb_gemm(mode, M, N, K, alpha, dA, lda, w, beta, dC, ldc, ws, need > 0 ? kScratchBytes : 0, stream);
}

/* The int8-table GEMM's split: at most a thousand rows whose 64 x 64 tiles leave CUs idle and K beyond one 1024-row
 * block split K at the blocks (one workgroup per tile and block, int32 partial sums, fold_splits folds the blocks in
 * order: the unsplit kernel's bits). Measured on MI355X at M = 375, 4096 -> 1024 (96 tiles): 14.2 against 21.3 us. */
static int q8b_splits(int M, int N, int K)
{
    const int cus = g_cus > 0 ? g_cus : 256;
    const long long tiles = (long long)((M + 63) / 64) * ((N + 63) / 64);
    return (M <= 1024 && K > p2k::kFoldRows && tiles < cus) ? (K + p2k::kFoldRows - 1) / p2k::kFoldRows : 1;
}

static size_t q8b_part_bytes(int M, int N, int K)
{
    const int sp = q8b_splits(M, N, K);
    return sp > 1 ? align_up((size_t)sp * M * N * 4, 256) : 0;
}

/* p2h_q8b_gemm_q8a after its checks (M, N, K > 0, alpha != 0); part: room for the split's partial sums, or null */
static int q8b_launch(int M, int N, int K, float alpha, const signed char *dQ, int ldq, const float *dScales,
                      const signed char *dB, int ldb, const float *dBscales, float beta, float *dC, int ldc,
                      void *part, size_t part_bytes, hipStream_t s)
{
    const int cus = g_cus > 0 ? g_cus : 256;
    const bool small = M <= 1024;   /* 64 x 64 tiles up to a thousand rows, 128 x 128 beyond */
    Plan p;
    memset(&p, 0, sizeof p);
    p.tiles_m = (M + (small ? 63 : 127)) / (small ? 64 : 128);
    p.tiles_n = (N + (small ? 63 : 127)) / (small ? 64 : 128);
    p.splits = 1;
    p.split_rows = K;
    const int sp = q8b_splits(M, N, K);
    /* K <= 1024 with idle CUs: 32 x 64 tiles, twice the workgroups (M = 375, 1024 -> 640: 5.9 against 7.6 us) */
    const bool narrow = small && K <= p2k::kFoldRows && (long long)p.tiles_m * p.tiles_n < cus;
    if (narrow) p.tiles_m = (M + G3264::BM - 1) / G3264::BM;
    if (sp > 1 && part && part_bytes >= q8b_part_bytes(M, N, K)) {
        p.splits = sp;
        p.split_rows = p2k::kFoldRows;
    }
    p2k::GemmArgs g = gemm_args(M, N, K, alpha, beta, dQ, ldq, dScales, dC, ldc, p, p.splits > 1 ? part : nullptr);
    g.B8 = (const int8_t *)dB; g.ldb = ldb; g.c1 = dBscales;
    const dim3 grid((unsigned)((size_t)p.tiles_m * p.tiles_n * p.splits)), block(G64::NT);
    if (p.splits > 1) {
        hipLaunchKernelGGL((p2k::gemm_i8<G64, p2k::MODE_Q8B, p2k::OUT_F32, false, true>), grid, block, 0, s, g);
        const size_t quads = (size_t)M * (N / 4);
        hipLaunchKernelGGL((p2k::fold_splits<false>), dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, s, g);
    } else if (narrow)
        hipLaunchKernelGGL((p2k::gemm_i8<G3264, p2k::MODE_Q8B, p2k::OUT_F32, false, false>), grid, block, 0, s, g);
    else if (small && K > p2k::kFoldRows)
        hipLaunchKernelGGL((p2k::gemm_i8<G64, p2k::MODE_Q8B, p2k::OUT_F32, true, false>), grid, block, 0, s, g);
    else if (small)
        hipLaunchKernelGGL((p2k::gemm_i8<G64, p2k::MODE_Q8B, p2k::OUT_F32, false, false>), grid, block, 0, s, g);
    else if (K > p2k::kFoldRows)
        hipLaunchKernelGGL((p2k::gemm_i8<G128, p2k::MODE_Q8B, p2k::OUT_F32, true, false>), grid, block, 0, s, g);
    else
        hipLaunchKernelGGL((p2k::gemm_i8<G128, p2k::MODE_Q8B, p2k::OUT_F32, false, false>), grid, block, 0, s, g);
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

int p2h_q8b_gemm_q8a(int M, int N, int K, float alpha, const signed char *dQ, int ldq, const float *dScales,
                     const signed char *dB, int ldb, const float *dBscales, float beta, float *dC, int ldc,
                     void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (N < 0 || N % 16 != 0) return fail(P2H_E_ARG, "p2h_q8b_gemm_q8a: N = %d is not a multiple of 16", N);
    if (int rc = check_q("p2h_q8b_gemm_q8a", M, K, dQ, ldq, dScales)) return rc;
    if (M > 0 && K > 0 && (!dB || !dBscales || ldb < N || ldb % 16 != 0 || !aligned(dB, 16)))
        return fail(P2H_E_ARG, "p2h_q8b_gemm_q8a: B must be 16-byte aligned with ldb %% 16 == 0 and ldb >= N");
    if (M > 0 && (!dC || ldc < N)) return fail(P2H_E_ARG, "p2h_q8b_gemm_q8a: C or ldc invalid");
    hipStream_t s = stream_of(stream);
    if (M == 0 || N == 0) return P2H_OK;
    if (alpha == 0.0f) return p2h_scale_c(M, N, beta, dC, ldc, s);
    if (K == 0) return (beta != 0.0f) ? p2h_scale_c(M, N, beta, dC, ldc, s) : P2H_OK;
    return q8b_launch(M, N, K, alpha, dQ, ldq, dScales, dB, ldb, dBscales, beta, dC, ldc, nullptr, 0, s);
}

size_t p2h_q8b_workspace_bytes(int mode, int M, int N, int K)
{
    if (ensure_init() || mode == P2H_EXACT || M <= 0 || N <= 0 || K <= 0 || K % 4 != 0) return 0;
    return quant_area(M, K) + q8b_part_bytes(M, N, K);
}

int p2h_q8b_gemm(int mode, int M, int N, int K, float alpha, const float *dA, int lda, const signed char *dB,
                 int ldb, const float *dBscales, float beta, float *dC, int ldc, void *workspace,
                 size_t workspace_bytes, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (mode != P2H_INT8W && mode != P2H_INT8 && mode != P2H_EXACT)
        return fail(P2H_E_ARG, "p2h_q8b_gemm: unknown mode %d", mode);
    if (N < 0 || N % 16 != 0) return fail(P2H_E_ARG, "p2h_q8b_gemm: N = %d is not a multiple of 16", N);
    if (M < 0 || K < 0) return fail(P2H_E_ARG, "p2h_q8b_gemm: negative shape");
    if (M > 0 && (!dC || ldc < N || (K > 0 && (!dA || lda < K || !dB || !dBscales || ldb < N))))
        return fail(P2H_E_ARG, "p2h_q8b_gemm: bad A/B/C");
    hipStream_t s = stream_of(stream);
    if (M == 0 || N == 0) return P2H_OK;
    if (alpha == 0.0f) return p2h_scale_c(M, N, beta, dC, ldc, s);
    if (mode != P2H_EXACT && K % 4 == 0) {   /* blas.c:1453-1457 */
        if (beta != 0.0f && beta != 1.0f) {
            if (int rc = p2h_scale_c(M, N, beta, dC, ldc, s)) return rc;
            beta = 1.0f;
        }
        if (K == 0) return P2H_OK;
        /* workspace: [quantised rows][row scales][the split's partial sums, when it has room for them] */
        const size_t qa = quant_area(M, K);
        if (!workspace || workspace_bytes < qa || !aligned(workspace, 256))
            return fail(P2H_E_WORKSPACE, "p2h_q8b_gemm: workspace of %zu bytes (256-byte aligned) needed, %zu given "
                        "(p2h_q8b_workspace_bytes: %zu with room to split K)", qa, workspace_bytes,
                        p2h_q8b_workspace_bytes(mode, M, N, K));
        if (ldb % 16 != 0 || !aligned(dB, 16))
            return fail(P2H_E_ARG, "p2h_q8b_gemm: B must be 16-byte aligned with ldb %% 16 == 0 and ldb >= N");
        signed char *dQ = (signed char *)workspace;
        float *dS = (float *)((char *)workspace + align_up(p2h_q_bytes(M, K), 256));
        if (int rc = p2h_quant_rows(M, K, dA, lda, dQ, p2h_q_ld(K), dS, s)) return rc;
        return q8b_launch(M, N, K, alpha, dQ, p2h_q_ld(K), dS, dB, ldb, dBscales, beta, dC, ldc,
                          (char *)workspace + qa, workspace_bytes - qa, s);
    }
    p2k::ExactArgs g;
    memset(&g, 0, sizeof g);
    g.M = M; g.N = N; g.K = K; g.alpha = alpha; g.beta = beta;
    g.A = dA; g.lda = lda;
    g.B8 = (const int8_t *)dB; g.ldb = ldb; g.bscales = dBscales;
    g.C = dC; g.ldc = ldc;
    return launch_exact(p2k::EXB_Q8, g, s);
}

int p2h_sgemm_batched(int transA, int transB, int M, int N, int K, float alpha, const float *dA, int lda,
                      long long strideA, const float *dB, int ldb, long long strideB, float beta, float *dC, int ldc,
                      long long strideC, int batch, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (M < 0 || N < 0 || K < 0 || batch < 0 || batch > 65535)
        return fail(P2H_E_ARG, "p2h_sgemm_batched: shape %d x %d x %d, batch %d", M, N, K, batch);
    if (M > 0 && N > 0 && batch > 0 && (!dC || ldc < N)) return fail(P2H_E_ARG, "p2h_sgemm: bad C");
    if (M > 0 && N > 0 && K > 0 && batch > 0 &&
        (!dA || !dB || lda < (transA ? M : K) || ldb < (transB ? K : N)))
        return fail(P2H_E_ARG, "p2h_sgemm: bad A/B");
    hipStream_t s = stream_of(stream);
    if (M == 0 || N == 0 || batch == 0) return P2H_OK;
    if (alpha == 0.0f || K == 0) {   /* blas.c:748-749 */
        for (int b = 0; b < batch; b++)
            if (int rc = p2h_scale_c(M, N, beta, dC + (size_t)b * strideC, ldc, s)) return rc;
        return P2H_OK;
    }
    p2k::SgemmArgs g;
    memset(&g, 0, sizeof g);
    g.M = M; g.N = N; g.K = K; g.alpha = alpha; g.beta = beta;
    g.A = dA; g.lda = lda; g.sA = strideA; g.transA = transA ? 1 : 0;
    g.B = dB; g.ldb = ldb; g.sB = strideB; g.transB = transB ? 1 : 0;
    g.C = dC; g.ldc = ldc; g.sC = strideC;
    g.tiles_n = (N + 63) / 64;
    g.batch = batch;
    const size_t blocks = (size_t)g.tiles_n * ((M + 63) / 64) * batch;
    if (blocks > 0x7fffffffu) return fail(P2H_E_ARG, "p2h_sgemm_batched: %zu tiles exceed one launch", blocks);
    const dim3 grid((unsigned)blocks);
    /* operand reads: 16-byte loads where every batch's rows are aligned and row lengths are multiples of 4, else
     * buffer loads (operands under 2 GiB), else element loads */
    const long long spanA = ((long long)((transA ? K : M) - 1) * lda + (transA ? M : K)) * 4;
    const long long spanB = ((long long)((transB ? N : K) - 1) * ldb + (transB ? K : N)) * 4;
    const bool va = lda % 4 == 0 && strideA % 4 == 0 && aligned(dA, 16) && (transA ? M : K) % 4 == 0;
    const bool vb = ldb % 4 == 0 && strideB % 4 == 0 && aligned(dB, 16) && (transB ? K : N) % 4 == 0;
    const bool small = spanA < (1ll << 31) && spanB < (1ll << 31);
    using VecT = std::integral_constant<int, p2k::LD_VEC>;
    using BufT = std::integral_constant<int, p2k::LD_BUF>;
    using AnyT = std::integral_constant<int, p2k::LD_ANY>;
    auto go = [&](auto ta, auto tb, auto la, auto lb) {
        hipLaunchKernelGGL((p2k::sgemm_f32<decltype(ta)::value, decltype(tb)::value, decltype(la)::value,
                                           decltype(lb)::value>),
                           grid, dim3(256), 0, s, g);
    };
    const bool any = !small || switch_of(g_sw.sgemm_any) != 0;   /* the variable forces the element loads (tests) */
    auto by_load = [&](auto ta, auto tb) {
        if (any) go(ta, tb, AnyT{}, AnyT{});
        else if (va && vb) go(ta, tb, VecT{}, VecT{});
        else if (va) go(ta, tb, VecT{}, BufT{});
        else if (vb) go(ta, tb, BufT{}, VecT{});
        else go(ta, tb, BufT{}, BufT{});
    };
    if (transA && transB) by_load(std::true_type{}, std::true_type{});
    else if (transA) by_load(std::true_type{}, std::false_type{});
    else if (transB) by_load(std::false_type{}, std::true_type{});
    else by_load(std::false_type{}, std::false_type{});
    HIPCHK(hipGetLastError());
    return P2H_OK;
}

int p2h_sgemm(int transA, int transB, int M, int N, int K, float alpha, const float *dA, int lda,
              const float *dB, int ldb, float beta, float *dC, int ldc, void *stream)
{
    return p2h_sgemm_batched(transA, transB, M, N, K, alpha, dA, lda, 0, dB, ldb, 0, beta, dC, ldc, 0, 1, stream);
}

/* ── one conformer block on the device ───────────────────────────────────────────────────────────────────────── */

namespace {

/* The block's buffers in the caller's workspace, 256-byte aligned sections. With base == nullptr only the size. */
struct BlockWs {
    signed char *q; float *sc;                   /* quantised rows [T][≤ 4096] and their scales (int8 modes) */
    float *h, *qkv, *qu, *qv, *p, *ac, *bd, *attn_h, *dw;
    float *ln, *out, *attn;                      /* exact mode: fp32 rows */
    void *gws; size_t gws_bytes;                 /* the GEMMs' own workspace */
    size_t total;
};

size_t gemm_ws_bytes(int mode, int T)
{
    const int D = p2k::kD, FF = 4 * p2k::kD, L = 2 * T - 1;
    const int shapes[6][2] = {{D, FF}, {FF, D}, {D, 3 * D}, {D, D}, {D, 2 * D}, {D, D}};
    size_t need = p2h_fvb_workspace_bytes(mode, L, D, D);   /* the positional rows go through the fp32-input GEMM */
    for (auto &sh : shapes) {
        need = std::max(need, mode == P2H_EXACT ? p2h_fvb_workspace_bytes(mode, T, sh[1], sh[0])
                                                : p2h_fvb_q8a_workspace_bytes(mode, T, sh[1], sh[0]));
    }
    return need;
}

BlockWs block_ws(int mode, int T, char *base)
{
    BlockWs w{};
    size_t off = 0;
    auto take = [&](size_t bytes) -> char * {
        char *p = base ? base + off : nullptr;
        off += align_up(bytes, 256);
        return p;
    };
    const size_t D = p2k::kD, Tz = (size_t)T, L = 2 * Tz - 1;
    if (mode != P2H_EXACT) {
        w.q = (signed char *)take(p2h_q_bytes(T, 4 * p2k::kD));
        w.sc = (float *)take(4 * Tz);
    } else {
        w.ln = (float *)take(4 * Tz * D);
        w.out = (float *)take(4 * Tz * D);
        w.attn = (float *)take(4 * Tz * D);
    }
    w.h = (float *)take(4 * Tz * 4 * D);
    w.qkv = (float *)take(4 * Tz * 3 * D);
    w.qu = (float *)take(4 * Tz * D);
    w.qv = (float *)take(4 * Tz * D);
    w.p = (float *)take(4 * L * D);
    w.ac = (float *)take(4 * p2k::kH * Tz * Tz);
    w.bd = (float *)take(4 * p2k::kH * Tz * L);
    w.attn_h = (float *)take(4 * Tz * D);
    w.dw = (float *)take(4 * D * Tz);
    w.gws_bytes = gemm_ws_bytes(mode, T);
    w.gws = w.gws_bytes ? take(w.gws_bytes) : nullptr;
    w.total = off;
    return w;
}

/* the fused attention kernel takes the block when its rows fit (T <= P2H_ATTENTION_TMAX) and the bias vectors are
 * 16-byte aligned; P2H_ATTENTION_FUSED=0 keeps the separate products (for comparisons) */
bool fused_attention(int T, const P2hBlock *blk)
{
    return T <= P2H_ATTENTION_TMAX && aligned(blk->bias_u, 16) && aligned(blk->bias_v, 16) &&
           switch_of(g_sw.attention_fused) != 0;
}

int check_block_weight(const P2hWeight *w, int K, int N, const char *name)
{
    if (!w || w->K != K || w->N != N)
        return fail(P2H_E_ARG, "p2h_conformer_block: %s must be a [%d, %d] five-value weight", name, K, N);
    return P2H_OK;
}

}  // namespace

size_t p2h_conformer_block_workspace_bytes(int mode, int T)
{
    if (ensure_init() || T <= 0 || (mode != P2H_INT8W && mode != P2H_INT8 && mode != P2H_EXACT)) return 0;
    return block_ws(mode, T, nullptr).total;
}

namespace {

/* the block's weights and vectors are present, of the shapes the reference's ConformerBlock holds */
int check_block(const P2hBlock *blk)
{
    const int D = p2k::kD, FF = 4 * p2k::kD;
    const struct { const P2hWeight *w; int K, N; const char *name; } lin[] = {
        {blk->ff1_l1, D, FF, "ff1_l1"}, {blk->ff1_l2, FF, D, "ff1_l2"}, {blk->qkv, D, 3 * D, "qkv"},
        {blk->pos, D, D, "pos"},        {blk->out, D, D, "out"},         {blk->pw1, D, 2 * D, "pw1"},
        {blk->pw2, D, D, "pw2"},        {blk->ff2_l1, D, FF, "ff2_l1"}, {blk->ff2_l2, FF, D, "ff2_l2"}};
    for (auto &x : lin)
        if (int rc = check_block_weight(x.w, x.K, x.N, x.name)) return rc;
    const float *vecs[] = {blk->norm_ff1_w, blk->norm_ff1_b, blk->norm_sa_w,   blk->norm_sa_b,   blk->bias_u,
                           blk->bias_v,     blk->norm_conv_w, blk->norm_conv_b, blk->dw_w,        blk->dw_b,
                           blk->norm_ff2_w, blk->norm_ff2_b, blk->norm_out_w,  blk->norm_out_b};
    for (const float *v : vecs)
        if (!v) return fail(P2H_E_ARG, "p2h_conformer_block: a null norm, bias or convolution vector");
    return P2H_OK;
}

/* one block on x in place (encoder.c:617-625); dP: its positional projection [2T − 1][1024] when the caller made
 * it, else null (made here from dPE). int8 modes, between the blocks of a stack: first_norm_done says that w.q /
 * w.sc already hold the int8 rows of this block's first LayerNorm (made with the previous block's output norm);
 * next, when set, has this block's output norm made together with next's first LayerNorm into w.q / w.sc. */
int run_block(int mode, const P2hBlock *blk, int T, const float *dPE, const float *dP, float *dX, const BlockWs &w,
              hipStream_t s, bool first_norm_done = false, const P2hBlock *next = nullptr)
{
    const int D = p2k::kD, FF = 4 * p2k::kD, L = 2 * T - 1, Dh = p2k::kDh, H = p2k::kH;
    const int ldD = p2h_q_ld(D), ldF = p2h_q_ld(FF);
#define P2H_TRY(call) do { if (int rc_ = (call)) return rc_; } while (0)
    /* a linear from produced rows: quantised (int8 modes) or fp32 (exact) */
    auto linear = [&](const P2hWeight *wt, int K, int N, float alpha, float beta, const float *rows, float *C) {
        if (mode == P2H_EXACT)
            return p2h_fvb_gemm(mode, T, N, K, alpha, rows, K, wt, beta, C, N, w.gws, w.gws_bytes, s);
        return p2h_fvb_gemm_q8a(mode, T, N, K, alpha, w.q, K > D ? ldF : ldD, w.sc, wt, beta, C, N, w.gws,
                                w.gws_bytes, s);
    };
    auto layer_norm = [&](const float *g, const float *b) {   /* x → the next linear's rows */
        if (mode == P2H_EXACT) return p2h_layer_norm_rows(T, D, dX, D, g, b, w.ln, D, s);
        return p2h_layer_norm_quant_rows(T, D, dX, D, g, b, w.q, ldD, w.sc, s);
    };
    const bool silu_epilogue = switch_of(g_sw.silu_epilogue) != 0;   /* 0: the SiLU→int8 producer instead */
    /* Exact mode's residuals (add_residual, encoder.c:252-275: x = fmaf(y, α, x) over y = the linear's output) in the
     * matrix-core GEMM's epilogue: fmaf(α, sum, x) with β = 1 is the same value, y being the sum itself (α = 1,
     * β = 0: fmaf(1, sum, 0)); only a −0 sum onto a −0 x would differ. The feed-forward's SiLU there too (see
     * exact_gemm). The fmaf-chain route (P2H_EXACT_CHAIN=1) keeps the separate passes, as the reference computes
     * them; so does P2H_EXACT_EPILOGUE=0. */
    const bool res_epilogue = mode == P2H_EXACT && switch_of(g_sw.exact_chain) == 0 &&
                              switch_of(g_sw.exact_epilogue) != 0;
    /* feed_forward (encoder.c:333-362): x += ½ · W2 · SiLU(W1 · LN(x)) */
    auto feed_forward = [&](const float *g, const float *b, const P2hWeight *l1, const P2hWeight *l2,
                            bool norm_done) {
        if (!norm_done) P2H_TRY(layer_norm(g, b));
        if (mode != P2H_EXACT && silu_epilogue) {   /* SiLU in the up-projection's epilogue, then the plain quantiser */
            P2H_TRY(fvb_gemm_q8a(mode, T, FF, D, 1.0f, w.q, ldD, w.sc, l1, 0.0f, w.h, FF, w.gws, w.gws_bytes,
                                 nullptr, s, true));
            P2H_TRY(p2h_quant_rows(T, FF, w.h, FF, w.q, ldF, w.sc, s));
        } else if (res_epilogue) {
            P2H_TRY(exact_gemm(T, FF, D, 1.0f, w.ln, D, l1, 0.0f, w.h, FF, s, true));
        } else {
            P2H_TRY(linear(l1, D, FF, 1.0f, 0.0f, w.ln, w.h));
            if (mode != P2H_EXACT) P2H_TRY(p2h_silu_quant_rows(T, FF, w.h, FF, w.q, ldF, w.sc, s));
            else P2H_TRY(p2h_silu((size_t)T * FF, w.h, s));
        }
        if (mode == P2H_EXACT) {
            if (res_epilogue) return linear(l2, FF, D, 0.5f, 1.0f, w.h, dX);
            P2H_TRY(linear(l2, FF, D, 1.0f, 0.0f, w.h, w.out));
            return p2h_add_residual(T, dX, w.out, 0.5f, s);
        }
        return linear(l2, FF, D, 0.5f, 1.0f, nullptr, dX);
    };
    P2H_TRY(feed_forward(blk->norm_ff1_w, blk->norm_ff1_b, blk->ff1_l1, blk->ff1_l2,
                         first_norm_done && mode != P2H_EXACT));
    /* self_attention (encoder.c:471-541) */
    P2H_TRY(layer_norm(blk->norm_sa_w, blk->norm_sa_b));
    P2H_TRY(linear(blk->qkv, D, 3 * D, 1.0f, 0.0f, w.ln, w.qkv));
    if (!dP) {   /* the positional projection, unless the caller made it (p2h_conformer_stack groups them) */
        P2H_TRY(p2h_fvb_gemm(mode, L, D, D, 1.0f, dPE, D, blk->pos, 0.0f, w.p, D, w.gws, w.gws_bytes, s));
        dP = w.p;
    }
    const bool fused = fused_attention(T, blk);
    if (fused) {   /* scores, shift, softmax and the product with V in one kernel, written as the heads' rows */
        P2H_TRY(p2h_attention_rows(T, w.qkv, blk->bias_u, blk->bias_v, dP, w.attn_h, s));
    } else {
        /* Q_u, Q_v as [H, T, Dh] (the bias adds of gather_heads); the products read K, V and the positional rows
         * where they lie, head h at column offset h·Dh of its row (the transposes of gather_heads and transpose_pos
         * are only layouts for the reference's NN kernel; the sums are the same) */
        hipLaunchKernelGGL(p2k::gather_qv, dim3((unsigned)(((size_t)T * D + 255) / 256)), dim3(256), 0, s, T, w.qkv,
                           blk->bias_u, blk->bias_v, w.qu, w.qv, (float *)nullptr);
        HIPCHK(hipGetLastError());
        P2H_TRY(p2h_sgemm_batched(0, 1, T, T, Dh, 1.0f, w.qu, Dh, (long long)T * Dh, w.qkv + D, 3 * D, Dh, 0.0f, w.ac,
                                  T, (long long)T * T, H, s));
        P2H_TRY(p2h_sgemm_batched(0, 1, T, L, Dh, 1.0f, w.qv, Dh, (long long)T * Dh, dP, D, Dh, 0.0f, w.bd, L,
                                  (long long)T * L, H, s));
        P2H_TRY(p2h_combine_softmax(T, w.ac, w.bd, s));
        P2H_TRY(p2h_sgemm_batched(0, 0, T, Dh, T, 1.0f, w.ac, T, (long long)T * T, w.qkv + 2 * D, 3 * D, Dh, 0.0f,
                                  w.attn_h, Dh, (long long)T * Dh, H, s));
    }
    /* w.attn_h: the heads' rows [T][1024] from the fused kernel, else [H][T][Dh] for the concatenation */
    if (mode == P2H_EXACT) {
        if (!fused) P2H_TRY(p2h_concat_heads_rows(T, w.attn_h, w.attn, s));
        if (res_epilogue) {
            P2H_TRY(linear(blk->out, D, D, 1.0f, 1.0f, fused ? w.attn_h : w.attn, dX));
        } else {
            P2H_TRY(linear(blk->out, D, D, 1.0f, 0.0f, fused ? w.attn_h : w.attn, w.out));
            P2H_TRY(p2h_add_residual(T, dX, w.out, 1.0f, s));
        }
    } else {
        if (fused) P2H_TRY(p2h_quant_rows(T, D, w.attn_h, D, w.q, ldD, w.sc, s));
        else P2H_TRY(p2h_concat_heads_quant_rows(H, T, Dh, w.attn_h, w.q, ldD, w.sc, s));
        P2H_TRY(linear(blk->out, D, D, 1.0f, 1.0f, nullptr, dX));
    }
    /* conv_module (encoder.c:573-613) */
    P2H_TRY(layer_norm(blk->norm_conv_w, blk->norm_conv_b));
    P2H_TRY(linear(blk->pw1, D, 2 * D, 1.0f, 0.0f, w.ln, w.h));
    /* the convolution's output as rows [T][1024] (channel_major_to_rows' transpose made by the kernel's stores); in
     * the int8 modes quantised in the same kernel, with no fp32 rows written */
    const bool conv_quant = mode != P2H_EXACT && switch_of(g_sw.conv_quant) != 0;
    if (conv_quant)
        P2H_TRY(p2h_glu_depthwise_conv_silu_quant_rows(T, w.h, blk->dw_w, blk->dw_b, w.q, ldD, w.sc, s));
    else
        P2H_TRY(p2h_glu_depthwise_conv_silu_rows(T, w.h, blk->dw_w, blk->dw_b, w.dw, s));
    if (mode == P2H_EXACT) {
        if (res_epilogue) {
            P2H_TRY(linear(blk->pw2, D, D, 1.0f, 1.0f, w.dw, dX));
        } else {
            P2H_TRY(linear(blk->pw2, D, D, 1.0f, 0.0f, w.dw, w.out));
            P2H_TRY(p2h_add_residual(T, dX, w.out, 1.0f, s));
        }
    } else {
        if (!conv_quant) P2H_TRY(p2h_quant_rows(T, D, w.dw, D, w.q, ldD, w.sc, s));
        P2H_TRY(linear(blk->pw2, D, D, 1.0f, 1.0f, nullptr, dX));
    }
    P2H_TRY(feed_forward(blk->norm_ff2_w, blk->norm_ff2_b, blk->ff2_l1, blk->ff2_l2, false));
    if (next && mode != P2H_EXACT)   /* x = LayerNorm(x), and the next block's first LayerNorm of it as int8 rows */
        P2H_TRY(p2h_layer_norm2_quant_rows(T, D, dX, D, blk->norm_out_w, blk->norm_out_b, dX, D, next->norm_ff1_w,
                                           next->norm_ff1_b, w.q, ldD, w.sc, s));
    else
        P2H_TRY(p2h_layer_norm_rows(T, D, dX, D, blk->norm_out_w, blk->norm_out_b, dX, D, s));
#undef P2H_TRY
    return P2H_OK;
}


}  // namespace

int p2h_conformer_block(int mode, const P2hBlock *blk, int T, const float *dPE, float *dX, void *workspace,
                        size_t workspace_bytes, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (mode != P2H_INT8W && mode != P2H_INT8 && mode != P2H_EXACT)
        return fail(P2H_E_ARG, "p2h_conformer_block: unknown mode %d", mode);
    if (T <= 0 || !blk || !dPE || !dX) return fail(P2H_E_ARG, "p2h_conformer_block: T = %d or a null pointer", T);
    if (int rc = check_block(blk)) return rc;
    const BlockWs need = block_ws(mode, T, nullptr);
    if (!workspace || workspace_bytes < need.total || !aligned(workspace, 256))
        return fail(P2H_E_WORKSPACE, "p2h_conformer_block: workspace of %zu bytes (256-byte aligned) needed",
                    need.total);
    return run_block(mode, blk, T, dPE, nullptr, dX, block_ws(mode, T, (char *)workspace), stream_of(stream));
}

/* The block stack (encode_blocks, encoder.c:628-644): the stack's workspace is one block's, then (int8 modes) the
 * n positional projections [n][2T − 1][1024] and the quantised positional rows. */
namespace {
struct StackWs {
    char *block; float *P; signed char *qpe; float *spe; size_t total;
};
StackWs stack_ws(int mode, int T, int n, char *base)
{
    StackWs s{};
    const size_t L = 2 * (size_t)T - 1, D = p2k::kD;
    size_t off = 0;
    auto take = [&](size_t bytes) -> char * {
        char *p = base ? base + off : nullptr;
        off += align_up(bytes, 256);
        return p;
    };
    s.block = take(block_ws(mode, T, nullptr).total);
    if (mode != P2H_EXACT) {
        s.P = (float *)take(4 * L * D * (size_t)n);
        s.qpe = (signed char *)take(p2h_q_bytes((int)L, (int)D));
        s.spe = (float *)take(4 * L);
    }
    s.total = off;
    return s;
}
}  // namespace

size_t p2h_conformer_stack_workspace_bytes(int mode, int T, int n_blocks)
{
    if (ensure_init() || T <= 0 || n_blocks <= 0 || (mode != P2H_INT8W && mode != P2H_INT8 && mode != P2H_EXACT))
        return 0;
    return stack_ws(mode, T, n_blocks, nullptr).total;
}

int p2h_conformer_stack(int mode, const P2hBlock *blocks, int n_blocks, int T, const float *dPE, float *dX,
                        void *workspace, size_t workspace_bytes, void *stream)
{
    if (int rc = ensure_init()) return rc;
    if (mode != P2H_INT8W && mode != P2H_INT8 && mode != P2H_EXACT)
        return fail(P2H_E_ARG, "p2h_conformer_stack: unknown mode %d", mode);
    if (T <= 0 || n_blocks < 0 || (n_blocks > 0 && !blocks) || !dPE || !dX)
        return fail(P2H_E_ARG, "p2h_conformer_stack: T = %d, %d blocks or a null pointer", T, n_blocks);
    if (n_blocks == 0) return P2H_OK;
    for (int b = 0; b < n_blocks; b++)
        if (int rc = check_block(&blocks[b])) return rc;
    const StackWs need = stack_ws(mode, T, n_blocks, nullptr);
    if (!workspace || workspace_bytes < need.total || !aligned(workspace, 256))
        return fail(P2H_E_WORKSPACE, "p2h_conformer_stack: workspace of %zu bytes (256-byte aligned) needed",
                    need.total);
    const StackWs sw = stack_ws(mode, T, n_blocks, (char *)workspace);
    const BlockWs w = block_ws(mode, T, sw.block);
    hipStream_t s = stream_of(stream);
    const int D = p2k::kD, L = 2 * T - 1;
    if (mode != P2H_EXACT) {
        /* the positional rows are the same for every block (encoder.c:630): quantised once, and the blocks'
         * projections of them in grouped launches, the same products the blocks would make one by one */
        const int ldq = p2h_q_ld(D);
        if (int rc = p2h_quant_rows(L, D, dPE, D, sw.qpe, ldq, sw.spe, s)) return rc;
        for (int b0 = 0; b0 < n_blocks; b0 += p2k::kMaxGroups) {
            const int g = std::min(p2k::kMaxGroups, n_blocks - b0);
            const P2hWeight *wq[p2k::kMaxGroups];
            float *cq[p2k::kMaxGroups];
            for (int q = 0; q < g; q++) {
                wq[q] = blocks[b0 + q].pos;
                cq[q] = sw.P + (size_t)(b0 + q) * L * D;
            }
            if (int rc = p2h_fvb_gemm_q8a_grouped(mode, L, D, D, 1.0f, sw.qpe, ldq, sw.spe, wq, g, 0.0f, cq, D, s))
                return rc;
        }
    }
    /* int8 modes: each block's output norm and the next block's first norm in one kernel */
    const bool pair_norms = mode != P2H_EXACT && switch_of(g_sw.stack_norm_pairs) != 0;
    for (int b = 0; b < n_blocks; b++) {
        const P2hBlock *next = pair_norms && b + 1 < n_blocks ? &blocks[b + 1] : nullptr;
        if (int rc = run_block(mode, &blocks[b], T, dPE, mode != P2H_EXACT ? sw.P + (size_t)b * L * D : nullptr, dX,
                               w, s, pair_norms && b > 0, next))
            return rc;
    }
    return P2H_OK;
}

}  // extern "C"
