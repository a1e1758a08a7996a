// jh_api.cpp -- the C ABI of libjunohip.so (declared in include/junohip.h).
//
// Host-side runtime around the kernels: shared per-device contexts
// (GpuContext.shared, GpuContext.java:109-120), device-resident packed
// matrices (DeviceHalfMatrix, DeviceHalfMatrix.java:41-115), per-thread HIP
// streams and pinned staging for the host-pointer calls (RocmMatVec's
// ThreadLocal stream / scratch, RocmMatVec.java:64-92), argument validation
// with the reference's messages, and a thread-local last-error string
// (GpuBindings.check, GpuBindings.java:180-183).
#include "../../include/junohip.h"

#include <hip/hip_runtime.h>

#include <dlfcn.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>

#include "jh_kernels.hpp"

struct jh_ctx {
    int device;
    int refs;
    int cu_count;
};

struct jh_qmat {
    jh_ctx *ctx;
    int type, rows, cols;
    size_t nbytes, pitch;
    uint8_t *d_raw;  // owned; nbytes + kTailPad bytes
};

// jh_gguf.cpp: with d_dst null only the tensor's geometry is returned.
int jh_gguf_stream_to_device(const jh_gguf *g, int64_t index, uint8_t *d_dst, int64_t *nbytes, int *type,
                             int64_t *rows, int64_t *cols);

namespace {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int ok() {
    g_last_error.clear();
    return JH_OK;
}

int hip_fail(const char *op, hipError_t rc) {
    return fail(JH_EHIP, "%s failed: rc=%d (%s)", op, (int)rc, hipGetErrorString(rc));
}

#define JH_HIP(op, expr)                                     \
    do {                                                     \
        hipError_t _rc = (expr);                             \
        if (_rc != hipSuccess) return hip_fail((op), _rc);   \
    } while (0)

// Test hook: JUNO_HIP_FAIL_ALLOC_AFTER=N makes every device allocation after
// the first N fail with JH_ENOMEM, so callers' CPU fallback can be exercised.
std::atomic<long> g_alloc_count{0};

long alloc_limit() {
    static long limit = [] {
        const char *v = getenv("JUNO_HIP_FAIL_ALLOC_AFTER");
        return v ? atol(v) : -1L;
    }();
    return limit;
}

int device_alloc(void **p, size_t bytes) {
    long lim = alloc_limit();
    if (lim >= 0 && g_alloc_count.fetch_add(1) >= lim)
        return fail(JH_ENOMEM, "hipMalloc failed: %zu bytes (JUNO_HIP_FAIL_ALLOC_AFTER=%ld)", bytes, lim);
    hipError_t rc = hipMalloc(p, bytes);
    if (rc != hipSuccess) {
        (void)hipGetLastError();
        return fail(JH_ENOMEM, "hipMalloc failed: %zu bytes: rc=%d (%s)", bytes, (int)rc, hipGetErrorString(rc));
    }
    return JH_OK;
}

bool type_geometry(int type, int *qk, int *bb) {
    switch (type) {
    case JH_TYPE_F32: *qk = 1; *bb = 4; return true;
    case JH_TYPE_Q8_0: *qk = 32; *bb = 34; return true;
    case JH_TYPE_Q2_K: *qk = 256; *bb = 84; return true;
    case JH_TYPE_Q3_K: *qk = 256; *bb = 110; return true;
    case JH_TYPE_Q4_K: *qk = 256; *bb = 144; return true;
    case JH_TYPE_Q5_K: *qk = 256; *bb = 176; return true;
    case JH_TYPE_Q6_K: *qk = 256; *bb = 210; return true;
    default: return false;
    }
}

// ---- shared contexts (one per device, reference counted)
std::mutex g_ctx_mu;
jh_ctx *g_ctx[64];

// ---- per-thread, per-device stream and staging
struct Staging {
    hipStream_t stream = nullptr;
    float *d_x = nullptr, *d_y = nullptr;
    size_t cap_x = 0, cap_y = 0;
    float *h_x = nullptr, *h_y = nullptr;  // pinned
    size_t cap_hx = 0, cap_hy = 0;
};

struct ThreadStaging {
    Staging per_dev[64];
    ~ThreadStaging() {
        for (auto &s : per_dev) {
            if (s.d_x) (void)hipFree(s.d_x);
            if (s.d_y) (void)hipFree(s.d_y);
            if (s.h_x) (void)hipHostFree(s.h_x);
            if (s.h_y) (void)hipHostFree(s.h_y);
            if (s.stream) (void)hipStreamDestroy(s.stream);
        }
    }
};
thread_local ThreadStaging t_staging;

int grow_dev(float **p, size_t *cap, size_t bytes) {
    if (*cap >= bytes) return JH_OK;
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
    size_t want = bytes < 4096 ? 4096 : bytes;
    int rc = device_alloc((void **)p, want);
    if (rc) return rc;
    *cap = want;
    return JH_OK;
}

int grow_host(float **p, size_t *cap, size_t bytes) {
    if (*cap >= bytes) return JH_OK;
    if (*p) (void)hipHostFree(*p);
    *p = nullptr;
    *cap = 0;
    size_t want = bytes < 4096 ? 4096 : bytes;
    JH_HIP("hipHostMalloc(staging)", hipHostMalloc((void **)p, want, hipHostMallocDefault));
    *cap = want;
    return JH_OK;
}

int staging_for(int device, size_t bx, size_t by, Staging **out) {
    Staging &s = t_staging.per_dev[device];
    if (!s.stream) JH_HIP("hipStreamCreateWithFlags", hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking));
    int rc;
    if ((rc = grow_dev(&s.d_x, &s.cap_x, bx)) || (rc = grow_dev(&s.d_y, &s.cap_y, by)) ||
        (rc = grow_host(&s.h_x, &s.cap_hx, bx)) || (rc = grow_host(&s.h_y, &s.cap_hy, by)))
        return rc;
    *out = &s;
    return JH_OK;
}

int check_qmat(const jh_qmat *m) {
    if (!m) return fail(JH_EINVAL, "A must not be null");
    if (!m->d_raw) return fail(JH_ECLOSED, "DeviceQuantMatrix is closed");
    return JH_OK;
}

int check_range(const jh_qmat *m, int row_start, int row_end) {
    if (row_start < 0 || row_end < row_start || row_end > m->rows)
        return fail(JH_EINVAL, "row range [%d, %d) outside rows=%d", row_start, row_end, m->rows);
    return JH_OK;
}

int gemv_path();

// Device workspace, one per (device, stream): the MFMA path's prepared x slabs
// and split-K partials, the attention partials, the LoRA intermediate.  Work
// on one stream is ordered, so a stream's launches never overlap in it.  One
// allocation holds the split-K arrival counters (kCounterSlots 128-byte-spaced
// ints, zeroed on the stream when allocated; every launch leaves them zero)
// followed by the scratch area.
//
// A HIP graph captured from calls on a stream keeps the addresses of that
// stream's workspace and counters.  So a buffer is never freed while the
// process runs: when a call needs more scratch than the stream has, a larger
// buffer (at least twice the old one, with fresh counters) replaces it for
// later calls, and the old one stays allocated, so that graphs captured
// earlier still replay into valid memory.  Growth is geometric, so the retired
// buffers total less than the live one.  Growth cannot happen inside a graph
// capture (no allocation may be recorded, and the counters' zeroing must not be
// a graph node): the call then fails and names the eager call to make first.
// A graph shares its stream's workspace: replaying it on another stream while
// work that uses the same workspace runs is a race, like any two overlapping
// launches on one buffer.
struct Workspace {
    uint8_t *base = nullptr;  // counters, then scratch
    size_t cap = 0;           // scratch bytes
};
constexpr size_t kCounterBytes = sizeof(int) * (size_t)jh::kCounterSlots * jh::kCounterStride;
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;

int stream_is_capturing(hipStream_t s, bool *capturing) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    JH_HIP("hipStreamIsCapturing", hipStreamIsCapturing(s, &st));
    *capturing = st != hipStreamCaptureStatusNone;
    return JH_OK;
}

// Scratch of at least `bytes` and the split-K counters of stream s on `device`.
int stream_workspace(int device, hipStream_t s, size_t bytes, void **out, int **counters = nullptr) {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Workspace &e = g_ws[{device, s}];
    if (!e.base || e.cap < bytes) {
        bool capturing = false;
        int rc = stream_is_capturing(s, &capturing);
        if (rc) return rc;
        if (capturing)
            return fail(JH_EINVAL,
                        "device workspace of %zu bytes needed during graph capture (stream has %zu): make one eager "
                        "call of the same size on this stream before capturing",
                        bytes, e.cap);
        size_t want = bytes < (8u << 20) ? (8u << 20) : bytes;
        if (e.base && want < 2 * e.cap) want = 2 * e.cap;
        void *p = nullptr;
        if ((rc = device_alloc(&p, kCounterBytes + want))) return rc;
        hipError_t me = hipMemsetAsync(p, 0, kCounterBytes, s);
        if (me != hipSuccess) {
            (void)hipFree(p);  // never handed out
            return hip_fail("hipMemsetAsync(split-K counters)", me);
        }
        // the previous buffer (if any) is retired, not freed: see above
        e.base = static_cast<uint8_t *>(p);
        e.cap = want;
    }
    *out = e.base + kCounterBytes;
    if (counters) *counters = reinterpret_cast<int *>(e.base);
    return JH_OK;
}

// The MFMA path for a group of matrices sharing K (B >= kMfmaMinBatch): kMfmaNotApplicable
// (never returned through the C ABI) when it does not apply, so that the caller
// can take the per-matrix kernels.
constexpr int kMfmaNotApplicable = -1;

int enqueue_mfma_group(int device, int n, const jh::MfmaDesc *d, int B, hipStream_t s) {
    const size_t wsb = jh::mfma_group_workspace_bytes(n, d, B);
    if (!wsb) return kMfmaNotApplicable;
    void *ws = nullptr;
    int *counters = nullptr;
    int rc = stream_workspace(device, s, wsb, &ws, &counters);
    if (rc) return rc;
    hipError_t e = jh::launch_mfma_group(n, d, B, ws, counters, s);
    if (e == hipSuccess) return JH_OK;
    if (e == hipErrorNotSupported) return kMfmaNotApplicable;
    return hip_fail("mfma_group launch", e);
}

// Enqueue y = W x for B vectors (device pointers), splitting B into the
// kernel's supported batch widths, or using the MFMA path for B >= kMfmaMinBatch.
int enqueue_matvec(const jh_qmat *m, const float *d_x, int B, float *d_y, int row_start, int row_end,
                   hipStream_t s, bool mfma = true) {
    const int nrows = row_end - row_start;
    if (nrows == 0 || B == 0) return JH_OK;
    jh::GemvArgs a;
    a.type = m->type;
    a.w = m->d_raw;
    a.pitch = m->pitch;
    a.cols = m->cols;
    a.row_start = row_start;
    a.row_end = row_end;
    a.ldx = m->cols;
    a.ldy = nrows;
    if (B >= jh::kMfmaMinBatch && mfma) {
        const jh::MfmaDesc d{m->type, m->d_raw, m->pitch, m->cols, row_start, row_end, d_x, d_y};
        int rc = enqueue_mfma_group(m->ctx->device, 1, &d, B, s);
        if (rc != kMfmaNotApplicable) return rc;
    }
    if (B == 1 && gemv_path() != 1) {
        a.batch = 1;
        a.x = d_x;
        a.y = d_y;
        hipError_t rc = jh::launch_gemv_staged(a, s);
        if (rc == hipSuccess) return JH_OK;
        if (rc != hipErrorNotSupported) return hip_fail("gemv_staged launch", rc);
    }
    int done = 0;
    while (done < B) {
        int left = B - done;
        int w = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
        a.batch = w;
        a.x = d_x + (size_t)done * m->cols;
        a.y = d_y + (size_t)done * nrows;
        hipError_t rc = jh::launch_gemv(a, s);
        if (rc != hipSuccess) return hip_fail("gemv launch", rc);
        done += w;
    }
    return JH_OK;
}

// JUNO_GEMV_PATH=basic forces the per-lane-block kernels of jh_gemv.hip for
// B = 1 (A/B measurements); the default uses the staged kernels where they apply.
int gemv_path() {
    static const int p = [] {
        const char *v = getenv("JUNO_GEMV_PATH");
        return (v && strcmp(v, "basic") == 0) ? 1 : 0;
    }();
    return p;
}

int set_device(int dev) {
    JH_HIP("hipSetDevice", hipSetDevice(dev));
    return JH_OK;
}

}  // namespace

extern "C" {

const char *jh_last_error(void) { return g_last_error.c_str(); }

int jh_qmatvec_batched_plan_shape(int ggml_type, int cols, int row_start, int row_end, int B, int *kernel,
                                  int *ksplit) {
    if (!kernel || !ksplit) return fail(JH_EINVAL, "kernel and ksplit must not be null");
    int qk, bb;
    if (!type_geometry(ggml_type, &qk, &bb)) return fail(JH_EUNSUPPORTED, "no block geometry for GGML type %d", ggml_type);
    if (cols <= 0 || cols % qk || row_start < 0 || row_end < row_start)
        return fail(JH_EINVAL, "invalid shape: cols=%d rows [%d, %d)", cols, row_start, row_end);
    // the planner reads formats, sizes and alignment only: a 256-byte-aligned stand-in address will do
    const uint8_t *w = reinterpret_cast<const uint8_t *>(uintptr_t(1) << 20);
    const jh::MfmaDesc d{ggml_type, w, (size_t)(cols / qk) * bb, cols, row_start, row_end,
                         reinterpret_cast<const float *>(w), nullptr};
    *ksplit = 1;
    *kernel = B >= jh::kMfmaMinBatch ? jh::mfma_group_plan(1, &d, B, ksplit) : 0;
    return ok();
}

int jh_qmatvec_batched_plan(int n, const jh_qmat *const *mats, int B, int *kernel, int *ksplit) {
    if (n < 1 || n > jh::kMaxMfmaGroup) return fail(JH_EINVAL, "n=%d outside [1, %d]", n, jh::kMaxMfmaGroup);
    if (!mats || !kernel || !ksplit) return fail(JH_EINVAL, "mats, kernel and ksplit must not be null");
    jh::MfmaDesc d[jh::kMaxMfmaGroup];
    int rc;
    for (int i = 0; i < n; i++) {
        if ((rc = check_qmat(mats[i]))) return rc;
        // x is only checked for 16-byte alignment: any aligned stand-in will do
        d[i] = jh::MfmaDesc{mats[i]->type, mats[i]->d_raw, mats[i]->pitch, mats[i]->cols, 0, mats[i]->rows,
                            reinterpret_cast<const float *>(mats[i]->d_raw), nullptr};
    }
    *ksplit = 1;
    *kernel = B >= jh::kMfmaMinBatch ? jh::mfma_group_plan(n, d, B, ksplit) : 0;
    return ok();
}

int jh_stream_workspace_info(int device, void *stream, size_t *scratch_bytes, void **base) {
    if (!scratch_bytes || !base) return fail(JH_EINVAL, "scratch_bytes and base must not be null");
    std::lock_guard<std::mutex> lk(g_ws_mu);
    auto it = g_ws.find({device, (hipStream_t)stream});
    *scratch_bytes = it == g_ws.end() ? 0 : it->second.cap;
    *base = it == g_ws.end() ? nullptr : it->second.base;
    return ok();
}

int jh_internal_fail(int code, const char *msg) {
    if (code == JH_OK) return ok();
    return fail(code, "%s", msg);
}

#ifndef JH_SRC_HASH
#define JH_SRC_HASH "unknown"
#endif
// The build (juno_amd/build.py) passes the hash of the sources it compiled, so a
// loader can refuse a library left from other sources.
const char *jh_version(void) { return "junohip 0.1 gfx950 src:" JH_SRC_HASH; }

int jh_device_count(int *count) {
    if (!count) return fail(JH_EINVAL, "count must not be null");
    int n = 0;
    hipError_t rc = hipGetDeviceCount(&n);
    if (rc != hipSuccess) {
        (void)hipGetLastError();
        *count = 0;
        return ok();
    }
    *count = n;
    return ok();
}

int jh_device_info(int device, char name[256], uint64_t *vram_bytes, char arch[64]) {
    hipDeviceProp_t p;
    JH_HIP("hipGetDeviceProperties", hipGetDeviceProperties(&p, device));
    if (name) snprintf(name, 256, "%s", p.name);
    if (vram_bytes) *vram_bytes = (uint64_t)p.totalGlobalMem;
    if (arch) snprintf(arch, 64, "%s", p.gcnArchName);
    return ok();
}

int jh_ctx_create(int device, jh_ctx **out) {
    if (!out) return fail(JH_EINVAL, "out must not be null");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
        (void)hipGetLastError();
        return fail(JH_ENODEV, "no HIP device available");
    }
    if (device < 0 || device >= n || device >= 64) return fail(JH_EINVAL, "device %d out of range (count=%d)", device, n);
    hipDeviceProp_t p;
    JH_HIP("hipGetDeviceProperties", hipGetDeviceProperties(&p, device));
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(JH_ENODEV, "device %d is %s; libjunohip is built for gfx950 only", device, p.gcnArchName);
    std::lock_guard<std::mutex> lk(g_ctx_mu);
    if (!g_ctx[device]) {
        int rc = set_device(device);
        if (rc) return rc;
        jh_ctx *c = new jh_ctx{device, 0, p.multiProcessorCount};
        g_ctx[device] = c;
    }
    g_ctx[device]->refs++;
    *out = g_ctx[device];
    return ok();
}

int jh_ctx_destroy(jh_ctx *ctx) {
    if (!ctx) return ok();
    std::lock_guard<std::mutex> lk(g_ctx_mu);
    // The shared context lives for the process, like GpuContext.shared; the
    // count only tracks users.
    if (ctx->refs > 0) ctx->refs--;
    return ok();
}

int jh_raw_byte_count(int type, int64_t nelems, int64_t *out) {
    int qk, bb;
    if (!type_geometry(type, &qk, &bb)) return fail(JH_EUNSUPPORTED, "No byte-size formula for GGML type %d", type);
    if (!out) return fail(JH_EINVAL, "out must not be null");
    // Java long arithmetic: the product wraps (two's complement) instead of
    // being undefined as a signed overflow in C++
    *out = (int64_t)((uint64_t)(nelems / qk) * (uint64_t)bb);
    return ok();
}

static int qmat_alloc(jh_ctx *ctx, int type, int rows, int cols, jh_qmat **out) {
    if (!ctx) return fail(JH_EINVAL, "ctx must not be null");
    if (!out) return fail(JH_EINVAL, "out must not be null");
    int qk, bb;
    if (!type_geometry(type, &qk, &bb))
        return fail(JH_EUNSUPPORTED, "Quantized matVec not implemented for GGML type %d", type);
    if (rows < 0 || cols <= 0) return fail(JH_EINVAL, "rows*cols invalid: rows=%d cols=%d", rows, cols);
    if (cols % qk) return fail(JH_EINVAL, "cols=%d is not a multiple of the block size %d", cols, qk);
    int rc = set_device(ctx->device);
    if (rc) return rc;
    jh_qmat *m = new jh_qmat;
    m->ctx = ctx;
    m->type = type;
    m->rows = rows;
    m->cols = cols;
    m->pitch = (size_t)(cols / qk) * bb;
    m->nbytes = m->pitch * (size_t)rows;
    m->d_raw = nullptr;
    rc = device_alloc((void **)&m->d_raw, m->nbytes + jh::kTailPad);
    if (rc) {
        delete m;
        return rc;
    }
    hipError_t e = hipMemset(m->d_raw + m->nbytes, 0, jh::kTailPad);
    if (e != hipSuccess) {
        (void)hipFree(m->d_raw);
        delete m;
        return hip_fail("hipMemset(pad)", e);
    }
    *out = m;
    return JH_OK;
}

int jh_qmat_upload(jh_ctx *ctx, int type, const void *raw, size_t nbytes, int rows, int cols, jh_qmat **out) {
    if (!raw && nbytes) return fail(JH_EINVAL, "raw must not be null");
    int qk, bb;
    if (type_geometry(type, &qk, &bb) && rows >= 0 && cols > 0 && cols % qk == 0) {
        size_t want = (size_t)(cols / qk) * bb * (size_t)rows;
        if (nbytes != want)
            return fail(JH_EINVAL, "raw.length=%zu != rawByteCount(type=%d, rows*cols=%lld)=%zu", nbytes, type,
                        (long long)rows * cols, want);
    }
    jh_qmat *m;
    int rc = qmat_alloc(ctx, type, rows, cols, &m);
    if (rc) return rc;
    hipError_t e = hipMemcpy(m->d_raw, raw, nbytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(m->d_raw);
        delete m;
        return hip_fail("hipMemcpy(raw H2D)", e);
    }
    *out = m;
    return ok();
}

int jh_qmat_quantize_dev(jh_ctx *ctx, int type, const float *d_src, int rows, int cols, void *stream,
                         jh_qmat **out) {
    if (!d_src && rows) return fail(JH_EINVAL, "src must not be null");
    jh_qmat *m;
    int rc = qmat_alloc(ctx, type, rows, cols, &m);
    if (rc) return rc;
    hipError_t e = jh::launch_quantize(type, d_src, (int64_t)rows * cols, m->d_raw, (hipStream_t)stream);
    if (e != hipSuccess) {
        (void)hipFree(m->d_raw);
        delete m;
        return hip_fail("quantize launch", e);
    }
    *out = m;
    return ok();
}

int jh_qmat_free(jh_qmat *m) {
    if (!m) return ok();
    if (m->d_raw) {
        (void)hipSetDevice(m->ctx->device);
        (void)hipFree(m->d_raw);
    }
    delete m;
    return ok();
}

int jh_qmat_info(const jh_qmat *m, int *type, int *rows, int *cols, size_t *nbytes, const void **d_raw) {
    if (!m) return fail(JH_EINVAL, "A must not be null");
    if (type) *type = m->type;
    if (rows) *rows = m->rows;
    if (cols) *cols = m->cols;
    if (nbytes) *nbytes = m->nbytes;
    if (d_raw) *d_raw = m->d_raw;
    return ok();
}

// ------------------------------------------------------------------ juno.MatVec ranges
// The reference wraps every matVec in a JFR event "juno.MatVec" with the backend
// label, rows and cols (MatVecEvent.java:46-72, MatVecBackend.java:36-64).  Here
// the same call sites push a roctx range "juno.MatVec backend=<label> rows=R
// cols=C batch=B" when JUNO_ROCTX=1 (rocprofv3 --marker-trace records them);
// the roctx library is opened at the first such call, so the library has no
// link-time dependency on it.  The range covers the host call: for the synchronous entry
// points that is the H2D copy, the kernels and the D2H copy, as the reference's
// event covers its transfers; for the _dev entry points it is the enqueue.
namespace {
typedef int (*roctx_push_t)(const char *);
typedef int (*roctx_pop_t)();
struct Roctx {
    roctx_push_t push = nullptr;
    roctx_pop_t pop = nullptr;
};
const Roctx &roctx() {
    static const Roctx r = [] {
        Roctx t;
        const char *e = getenv("JUNO_ROCTX");
        if (!e || strcmp(e, "1") != 0) return t;
        // rocprofv3 intercepts the rocprofiler-sdk roctx library; the older
        // roctracer one (libroctx64) serves roctracer-based tools
        void *h = nullptr;
        for (const char *lib : {"librocprofiler-sdk-roctx.so.1", "/opt/rocm/lib/librocprofiler-sdk-roctx.so.1",
                                "libroctx64.so", "/opt/rocm/lib/libroctx64.so"})
            if (!h) h = dlopen(lib, RTLD_NOW | RTLD_LOCAL);
        if (!h) return t;
        t.push = reinterpret_cast<roctx_push_t>(dlsym(h, "roctxRangePushA"));
        t.pop = reinterpret_cast<roctx_pop_t>(dlsym(h, "roctxRangePop"));
        if (!t.push || !t.pop) t.push = nullptr, t.pop = nullptr;
        return t;
    }();
    return r;
}
// MatVecBackend labels of the resident quantized matrices (juno_amd/matvec.py MatVecBackend.for_type)
const char *backend_label(int type) {
    switch (type) {
    case JH_TYPE_F32: return "rocm-resident";
    case 10: return "rocm-resident-q2k";
    case 11: return "rocm-resident-q3k";
    case 12: return "rocm-resident-q4k";
    case 13: return "rocm-resident-q5k";
    case 14: return "rocm-resident-q6k";
    case 8: return "rocm-resident-q8_0";
    default: return "rocm-resident";
    }
}
struct MatVecRange {
    bool on = false;
    MatVecRange(const char *backend, long long rows, long long cols, int batch) {
        const Roctx &r = roctx();
        if (!r.push) return;
        char msg[160];
        snprintf(msg, sizeof msg, "juno.MatVec backend=%s rows=%lld cols=%lld batch=%d", backend, rows, cols, batch);
        r.push(msg);
        on = true;
    }
    ~MatVecRange() {
        if (on) roctx().pop();
    }
};
}  // namespace

int jh_qmatvec_batched(jh_ctx *ctx, const jh_qmat *m, const float *X, int B, float *Y, int row_start, int row_end) {
    const MatVecRange range(m ? backend_label(m->type) : "rocm-resident", (long long)row_end - row_start,
                            m ? m->cols : 0, B);
    int rc;
    if (!ctx) return fail(JH_EINVAL, "ctx must not be null");
    if ((rc = check_qmat(m)) || (rc = check_range(m, row_start, row_end))) return rc;
    if (B < 0) return fail(JH_EINVAL, "B=%d must be >= 0", B);
    if ((!X || !Y) && B > 0) return fail(JH_EINVAL, "x and y must not be null");
    const int nrows = row_end - row_start;
    if (B == 0 || nrows == 0) return ok();
    if ((rc = set_device(ctx->device))) return rc;
    const size_t bx = (size_t)B * m->cols * 4, by = (size_t)B * nrows * 4;
    Staging *s;
    if ((rc = staging_for(ctx->device, bx, by, &s))) return rc;
    memcpy(s->h_x, X, bx);
    JH_HIP("hipMemcpyAsync(x H2D)", hipMemcpyAsync(s->d_x, s->h_x, bx, hipMemcpyHostToDevice, s->stream));
    if ((rc = enqueue_matvec(m, s->d_x, B, s->d_y, row_start, row_end, s->stream))) return rc;
    JH_HIP("hipMemcpyAsync(y D2H)", hipMemcpyAsync(s->h_y, s->d_y, by, hipMemcpyDeviceToHost, s->stream));
    JH_HIP("hipStreamSynchronize", hipStreamSynchronize(s->stream));
    memcpy(Y, s->h_y, by);
    return ok();
}

int jh_qmatvec(jh_ctx *ctx, const jh_qmat *m, const float *x, float *y, int row_start, int row_end) {
    return jh_qmatvec_batched(ctx, m, x, 1, y, row_start, row_end);
}

int jh_qmat_dequant(jh_ctx *ctx, const jh_qmat *m, float *out) {
    int rc;
    if (!ctx) return fail(JH_EINVAL, "ctx must not be null");
    if ((rc = check_qmat(m))) return rc;
    if (!out && m->rows) return fail(JH_EINVAL, "out must not be null");
    if ((rc = set_device(ctx->device))) return rc;
    const size_t bytes = (size_t)m->rows * m->cols * 4;
    if (bytes == 0) return ok();
    float *d_out = nullptr;
    if ((rc = device_alloc((void **)&d_out, bytes))) return rc;
    Staging *s;
    if ((rc = staging_for(ctx->device, 0, 0, &s))) {
        (void)hipFree(d_out);
        return rc;
    }
    hipError_t e = jh::launch_dequant(m->type, m->d_raw, m->rows, m->cols, d_out, s->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(out, d_out, bytes, hipMemcpyDeviceToHost, s->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    (void)hipFree(d_out);
    if (e != hipSuccess) return hip_fail("dequant", e);
    return ok();
}

int jh_sgemv(jh_ctx *ctx, const float *A, const float *x, int rows, int cols, float *y) {
    // MatVec contract (MatVec.java:46-54, MatVecBackendContractTest.java:196-212).
    if (!ctx) return fail(JH_EINVAL, "ctx must not be null");
    if (rows < 0 || cols <= 0) return fail(JH_EINVAL, "invalid shape: rows*cols with rows=%d cols=%d", rows, cols);
    if (!A || !x || !y) return fail(JH_EINVAL, "A, x and y must not be null");
    jh_qmat *m;
    int rc = jh_qmat_upload(ctx, JH_TYPE_F32, A, (size_t)rows * cols * 4, rows, cols, &m);
    if (rc) return rc;
    rc = jh_qmatvec(ctx, m, x, y, 0, rows);
    std::string err = g_last_error;
    jh_qmat_free(m);
    g_last_error = err;
    return rc;
}

int jh_qmatvec_dev(const jh_qmat *m, const float *d_x, float *d_y, int row_start, int row_end, void *stream) {
    return jh_qmatvec_batched_dev(m, d_x, 1, d_y, row_start, row_end, stream);
}

int jh_qmatvec_batched_dev(const jh_qmat *m, const float *d_X, int B, float *d_Y, int row_start, int row_end,
                           void *stream) {
    const MatVecRange range(m ? backend_label(m->type) : "rocm-resident", (long long)row_end - row_start,
                            m ? m->cols : 0, B);
    int rc;
    if ((rc = check_qmat(m)) || (rc = check_range(m, row_start, row_end))) return rc;
    if (B < 0) return fail(JH_EINVAL, "B=%d must be >= 0", B);
    if ((!d_X || !d_Y) && B > 0 && row_end > row_start) return fail(JH_EINVAL, "x and y must not be null");
    if ((rc = enqueue_matvec(m, d_X, B, d_Y, row_start, row_end, (hipStream_t)stream))) return rc;
    return ok();
}

int jh_qmatvec_batched_noalloc_dev(const jh_qmat *m, const float *d_X, int B, float *d_Y, int row_start, int row_end,
                                   void *stream) {
    int rc;
    if ((rc = check_qmat(m)) || (rc = check_range(m, row_start, row_end))) return rc;
    if (B < 0) return fail(JH_EINVAL, "B=%d must be >= 0", B);
    if (B == 0 || row_end == row_start) return ok();
    if (!d_X || !d_Y) return fail(JH_EINVAL, "x and y must not be null");
    if ((rc = set_device(m->ctx->device))) return rc;
    hipStream_t s = (hipStream_t)stream;
    if (B >= jh::kMfmaMinBatch) {
        const jh::MfmaDesc d{m->type, m->d_raw, m->pitch, m->cols, row_start, row_end, d_X, d_Y};
        const size_t wsb = jh::mfma_group_workspace_bytes(1, &d, B);
        if (wsb) {
            if (wsb > jh::kStaticScratchBytes)
                return fail(JH_EINVAL,
                            "rows=%d cols=%d B=%d needs %zu bytes of scratch; the static scratch holds %zu "
                            "(jh_qmatvec_batched_dev has no such limit)",
                            row_end - row_start, m->cols, B, wsb, jh::kStaticScratchBytes);
            void *ws = nullptr;
            int *counters = nullptr;
            hipError_t e = jh::static_scratch(m->ctx->device, s, &ws, &counters);
            if (e != hipSuccess) return hip_fail("static scratch (hipGetSymbolAddress)", e);
            e = jh::launch_mfma_group(1, &d, B, ws, counters, s);
            if (e == hipSuccess) return ok();
            if (e != hipErrorNotSupported) return hip_fail("mfma_group launch", e);
        }
    }
    // the kernels of the other batch sizes use no scratch
    if ((rc = enqueue_matvec(m, d_X, B, d_Y, row_start, row_end, s, false))) return rc;
    return ok();
}

int jh_qmatvec_group_dev(int n, const jh_qmat *const *mats, const float *const *d_x, float *const *d_y,
                         void *stream) {
    if (n < 0 || n > jh::kMaxGroup) return fail(JH_EINVAL, "n=%d outside [0, %d]", n, jh::kMaxGroup);
    if (n == 0) return ok();
    if (!mats || !d_x || !d_y) return fail(JH_EINVAL, "mats, x and y must not be null");
    long long grows = 0;
    for (int i = 0; i < n; i++) grows += mats[i] ? mats[i]->rows : 0;
    const MatVecRange range("rocm-resident-group", grows, mats[0] ? mats[0]->cols : 0, 1);
    jh::GroupProblem all[jh::kMaxGroup];
    int rc;
    for (int i = 0; i < n; i++) {
        if ((rc = check_qmat(mats[i]))) return rc;
        if (!d_x[i] || !d_y[i]) return fail(JH_EINVAL, "x[%d] and y[%d] must not be null", i, i);
        all[i] = jh::GroupProblem{mats[i]->type, mats[i]->d_raw, mats[i]->pitch, mats[i]->cols, mats[i]->rows,
                                  d_x[i], d_y[i], 0, 0};
    }
    hipStream_t s = (hipStream_t)stream;
    bool done[jh::kMaxGroup] = {};
    // 1. large same-format matrices sharing an x: one staged launch per class
    for (int i = 0; i < n; i++) {
        if (done[i] || all[i].type == JH_TYPE_F32 || gemv_path() == 1) continue;
        jh::GroupProblem cls[jh::kMaxStagedGroup];
        int idx[jh::kMaxStagedGroup], k = 0;
        for (int j = i; j < n && k < jh::kMaxStagedGroup; j++)
            if (!done[j] && all[j].type == all[i].type && all[j].cols == all[i].cols && all[j].x == all[i].x) {
                idx[k] = j;
                cls[k++] = all[j];
            }
        hipError_t e = jh::launch_gemv_staged_group(k, cls, s);
        if (e == hipSuccess) {
            for (int q = 0; q < k; q++) done[idx[q]] = true;
        } else if (e != hipErrorNotSupported) {
            return hip_fail("gemv_staged_group launch", e);
        }
    }
    // 2. everything else in one launch of the one-shot kernels (F32 on its own)
    jh::GroupArgs g = {};
    for (int i = 0; i < n; i++) {
        if (done[i]) continue;
        if (all[i].type == JH_TYPE_F32) {
            if ((rc = enqueue_matvec(mats[i], d_x[i], 1, d_y[i], 0, mats[i]->rows, s))) return rc;
            continue;
        }
        g.p[g.n++] = all[i];
    }
    if (g.n) {
        hipError_t e = jh::launch_gemv_group(g, s);
        if (e != hipSuccess) return hip_fail("gemv_group launch", e);
    }
    return ok();
}

int jh_qmatvec_swiglu_dev(const jh_qmat *gate, const jh_qmat *up, const float *d_x, float *d_out, void *stream) {
    int rc;
    if ((rc = check_qmat(gate)) || (rc = check_qmat(up))) return rc;
    if (!d_x || !d_out) return fail(JH_EINVAL, "x and out must not be null");
    if (gate->rows != up->rows || gate->cols != up->cols)
        return fail(JH_EINVAL, "gate [%d x %d] and up [%d x %d] differ in shape", gate->rows, gate->cols, up->rows,
                    up->cols);
    if (gate->ctx->device != up->ctx->device) return fail(JH_EINVAL, "matrices on different devices");
    hipStream_t s = (hipStream_t)stream;
    const jh::GroupProblem g{gate->type, gate->d_raw, gate->pitch, gate->cols, gate->rows, d_x, nullptr, 0, 0};
    const jh::GroupProblem u{up->type, up->d_raw, up->pitch, up->cols, up->rows, d_x, nullptr, 0, 0};
    if (gate->type != JH_TYPE_F32 && gemv_path() != 1) {
        hipError_t e = jh::launch_gemv_swiglu(g, u, d_out, s);
        if (e == hipSuccess) return ok();
        if (e != hipErrorNotSupported) return hip_fail("gemv_swiglu launch", e);
    }
    // the two projections into the stream's workspace, then the product
    void *ws = nullptr;
    if ((rc = stream_workspace(gate->ctx->device, s, 2 * sizeof(float) * (size_t)gate->rows, &ws))) return rc;
    float *yg = static_cast<float *>(ws), *yu = yg + gate->rows;
    const jh_qmat *mats[2] = {gate, up};
    const float *xs[2] = {d_x, d_x};
    float *ys[2] = {yg, yu};
    if ((rc = jh_qmatvec_group_dev(2, mats, xs, ys, stream))) return rc;
    hipError_t e = jh::launch_silu_mul(yg, yu, gate->rows, d_out, s);
    if (e != hipSuccess) return hip_fail("silu_mul launch", e);
    return ok();
}

int jh_debug_timeline(int device, int kernel, uint64_t *out, size_t n) {
    if (!out && n) return fail(JH_EINVAL, "out must not be null");
    if (kernel != 0 && kernel != 1) return fail(JH_EINVAL, "kernel=%d: 0 (staged walk) or 1 (batched MFMA)", kernel);
    int rc;
    if ((rc = set_device(device))) return rc;
    const hipError_t e = kernel == 0 ? jh::timeline_read(reinterpret_cast<unsigned long long *>(out), n)
                                     : jh::mfma_timeline_read(reinterpret_cast<unsigned long long *>(out), n);
    if (e == hipErrorNotSupported) return fail(JH_EUNSUPPORTED, "not a timeline build (-DJH_TIMELINE)");
    if (e != hipSuccess) return hip_fail("timeline read", e);
    return ok();
}

int jh_sync_faults(int device, unsigned int *count) {
    if (!count) return fail(JH_EINVAL, "count must not be null");
    int rc;
    if ((rc = set_device(device))) return rc;
    const hipError_t e = jh::sync_faults(count);
    if (e != hipSuccess) return hip_fail("sync_faults", e);
    return ok();
}

static int check_norm_args(const float *d_x, const float *d_res, const float *d_norm_w, const float *d_x_out,
                           const float *d_xn, int n) {
    if (!d_x || !d_norm_w || !d_xn) return fail(JH_EINVAL, "x, norm weights and xn scratch must not be null");
    if (n < 1 || n > (1 << 20)) return fail(JH_EINVAL, "n=%d outside [1, 2^20]", n);
    if (d_x_out && (d_x_out == d_x || d_x_out == d_res))
        return fail(JH_EINVAL, "x_out must not alias x or res (other workgroups still read them)");
    if (d_xn == d_x || d_xn == d_res || (d_x_out && d_xn == d_x_out)) return fail(JH_EINVAL, "xn must not alias x, res or x_out");
    return JH_OK;
}

int jh_rmsnorm_qmatvec_swiglu_dev(const jh_qmat *gate, const jh_qmat *up, const float *d_x, const float *d_res,
                                  const float *d_norm_w, float eps, float *d_x_out, float *d_xn, float *d_out,
                                  void *stream) {
    int rc;
    if ((rc = check_qmat(gate)) || (rc = check_qmat(up))) return rc;
    if (gate->rows != up->rows || gate->cols != up->cols)
        return fail(JH_EINVAL, "gate [%d x %d] and up [%d x %d] differ in shape", gate->rows, gate->cols, up->rows,
                    up->cols);
    if (!d_out) return fail(JH_EINVAL, "out must not be null");
    if ((rc = check_norm_args(d_x, d_res, d_norm_w, d_x_out, d_xn, gate->cols))) return rc;
    hipStream_t s = (hipStream_t)stream;
    if (d_res && gate->type != JH_TYPE_F32 && gemv_path() != 1) {
        const jh::GroupProblem g{gate->type, gate->d_raw, gate->pitch, gate->cols, gate->rows, d_x, nullptr, 0, 0};
        const jh::GroupProblem u{up->type, up->d_raw, up->pitch, up->cols, up->rows, d_x, nullptr, 0, 0};
        const jh::NormSpec ns{d_res, d_norm_w, eps, d_x_out};
        hipError_t e = jh::launch_gemv_swiglu(g, u, d_out, s, &ns);
        if (e == hipSuccess) return ok();
        if (e != hipErrorNotSupported) return hip_fail("gemv_swiglu (rmsnorm) launch", e);
    }
    if ((rc = jh_rmsnorm_dev(d_x, d_res, d_norm_w, gate->cols, eps, d_x_out, d_xn, stream))) return rc;
    return jh_qmatvec_swiglu_dev(gate, up, d_xn, d_out, stream);
}

int jh_rmsnorm_qmatvec_dev(const jh_qmat *m, const float *d_x, const float *d_res, const float *d_norm_w, float eps,
                           float *d_x_out, float *d_xn, float *d_y, void *stream) {
    int rc;
    if ((rc = check_qmat(m))) return rc;
    if (!d_y) return fail(JH_EINVAL, "y must not be null");
    if ((rc = check_norm_args(d_x, d_res, d_norm_w, d_x_out, d_xn, m->cols))) return rc;
    hipStream_t s = (hipStream_t)stream;
    if (d_res && m->type != JH_TYPE_F32 && gemv_path() != 1) {
        jh::GemvArgs a;
        a.type = m->type;
        a.w = m->d_raw;
        a.pitch = m->pitch;
        a.cols = m->cols;
        a.row_start = 0;
        a.row_end = m->rows;
        a.batch = 1;
        a.x = d_x;
        a.ldx = m->cols;
        a.y = d_y;
        a.ldy = m->rows;
        const jh::NormSpec ns{d_res, d_norm_w, eps, d_x_out};
        hipError_t e = jh::launch_gemv_staged(a, s, &ns);
        if (e == hipSuccess) return ok();
        if (e != hipErrorNotSupported) return hip_fail("gemv_staged (rmsnorm) launch", e);
    }
    if ((rc = jh_rmsnorm_dev(d_x, d_res, d_norm_w, m->cols, eps, d_x_out, d_xn, stream))) return rc;
    return jh_qmatvec_dev(m, d_xn, d_y, 0, m->rows, stream);
}

int jh_rmsnorm_qmatvec_group_dev(int n, const jh_qmat *const *mats, const float *d_x, const float *d_res,
                                 const float *d_norm_w, float eps, float *d_x_out, float *d_xn, float *const *d_y,
                                 void *stream) {
    if (n < 1 || n > jh::kMaxGroup) return fail(JH_EINVAL, "n=%d outside [1, %d]", n, jh::kMaxGroup);
    if (!mats || !d_y) return fail(JH_EINVAL, "mats and y must not be null");
    int rc;
    for (int i = 0; i < n; i++) {
        if ((rc = check_qmat(mats[i]))) return rc;
        if (!d_y[i]) return fail(JH_EINVAL, "y[%d] must not be null", i);
        if (mats[i]->cols != mats[0]->cols)
            return fail(JH_EINVAL, "matrix %d has %d columns, matrix 0 has %d (one input for all)", i, mats[i]->cols,
                        mats[0]->cols);
        if (mats[i]->ctx->device != mats[0]->ctx->device) return fail(JH_EINVAL, "matrices on different devices");
    }
    const int cols = mats[0]->cols;
    if ((rc = check_norm_args(d_x, d_res, d_norm_w, d_x_out, d_xn, cols))) return rc;
    hipStream_t s = (hipStream_t)stream;
    bool fused = d_res && gemv_path() != 1;
    for (int i = 0; i < n; i++) fused = fused && mats[i]->type != JH_TYPE_F32;
    if (fused) {
        jh::GroupArgs g = {};
        for (int i = 0; i < n; i++)
            g.p[g.n++] = jh::GroupProblem{mats[i]->type, mats[i]->d_raw, mats[i]->pitch, cols, mats[i]->rows, d_x,
                                          d_y[i], 0, 0};
        g.res = d_res;
        g.norm_w = d_norm_w;
        g.eps = eps;
        g.x_out = d_x_out;
        hipError_t e = jh::launch_gemv_group(g, s);
        if (e == hipSuccess) return ok();
        if (e != hipErrorNotSupported) return hip_fail("gemv_group (rmsnorm) launch", e);
    }
    if ((rc = jh_rmsnorm_dev(d_x, d_res, d_norm_w, cols, eps, d_x_out, d_xn, stream))) return rc;
    const float *xs[jh::kMaxGroup];
    for (int i = 0; i < n; i++) xs[i] = d_xn;
    return jh_qmatvec_group_dev(n, mats, xs, d_y, stream);
}

int jh_qmatvec_batched_swiglu_dev(const jh_qmat *gate, const jh_qmat *up, const float *d_X, int B, float *d_out,
                                  float *d_gate, float *d_up, void *stream) {
    int rc;
    if ((rc = check_qmat(gate)) || (rc = check_qmat(up))) return rc;
    if (B < 0) return fail(JH_EINVAL, "B=%d must be >= 0", B);
    if (B == 0) return ok();
    if (!d_X || !d_out) return fail(JH_EINVAL, "X and out must not be null");
    if (gate->rows != up->rows || gate->cols != up->cols)
        return fail(JH_EINVAL, "gate [%d x %d] and up [%d x %d] differ in shape", gate->rows, gate->cols, up->rows,
                    up->cols);
    if (gate->ctx->device != up->ctx->device) return fail(JH_EINVAL, "matrices on different devices");
    if (B == 1) return jh_qmatvec_swiglu_dev(gate, up, d_X, d_out, stream);
    hipStream_t s = (hipStream_t)stream;
    const jh::MfmaDesc dg{gate->type, gate->d_raw, gate->pitch, gate->cols, 0, gate->rows, d_X, nullptr};
    const jh::MfmaDesc du{up->type, up->d_raw, up->pitch, up->cols, 0, up->rows, d_X, nullptr};
    if (jh::mfma_swiglu_applies(dg, du, B)) {
        const int dev = gate->ctx->device;
        void *ws = nullptr;
        int *counters = nullptr;
        if ((rc = stream_workspace(dev, s, jh::mfma_swiglu_workspace_bytes(dg, B), &ws, &counters))) return rc;
        hipError_t e = jh::launch_mfma_swiglu(dg, du, B, d_out, ws, counters, s);
        if (e == hipSuccess) return ok();
        if (e != hipErrorNotSupported) return hip_fail("mfma swiglu launch", e);
    }
    if (!d_gate || !d_up) return fail(JH_EINVAL, "gate and up scratch must not be null on this path (B=%d)", B);
    const jh_qmat *mats[2] = {gate, up};
    const float *xs[2] = {d_X, d_X};
    float *ys[2] = {d_gate, d_up};
    if ((rc = jh_qmatvec_batched_group_dev(2, mats, xs, B, ys, stream))) return rc;
    hipError_t e = jh::launch_silu_mul(d_gate, d_up, B * gate->rows, d_out, s);
    if (e != hipSuccess) return hip_fail("silu_mul launch", e);
    return ok();
}

int jh_qmatvec_batched_group_dev(int n, const jh_qmat *const *mats, const float *const *d_X, int B,
                                 float *const *d_Y, void *stream) {
    if (n < 0 || n > jh::kMaxMfmaGroup) return fail(JH_EINVAL, "n=%d outside [0, %d]", n, jh::kMaxMfmaGroup);
    if (B < 0) return fail(JH_EINVAL, "B=%d must be >= 0", B);
    if (n == 0 || B == 0) return ok();
    if (!mats || !d_X || !d_Y) return fail(JH_EINVAL, "mats, X and Y must not be null");
    long long grows = 0;
    for (int i = 0; i < n; i++) grows += mats[i] ? mats[i]->rows : 0;
    const MatVecRange range("rocm-resident-group", grows, mats[0] ? mats[0]->cols : 0, B);
    int rc;
    jh::MfmaDesc d[jh::kMaxMfmaGroup];
    for (int i = 0; i < n; i++) {
        if ((rc = check_qmat(mats[i]))) return rc;
        if (!d_X[i] || !d_Y[i]) return fail(JH_EINVAL, "X[%d] and Y[%d] must not be null", i, i);
        if (mats[i]->ctx->device != mats[0]->ctx->device) return fail(JH_EINVAL, "matrices on different devices");
        d[i] = jh::MfmaDesc{mats[i]->type, mats[i]->d_raw, mats[i]->pitch, mats[i]->cols, 0, mats[i]->rows, d_X[i], d_Y[i]};
    }
    hipStream_t s = (hipStream_t)stream;
    if (B >= jh::kMfmaMinBatch) {
        rc = enqueue_mfma_group(mats[0]->ctx->device, n, d, B, s);
        if (rc != kMfmaNotApplicable) return rc ? rc : ok();
    }
    for (int i = 0; i < n; i++)
        if ((rc = enqueue_matvec(mats[i], d_X[i], B, d_Y[i], 0, mats[i]->rows, s))) return rc;
    return ok();
}

int jh_qmat_dequant_dev(const jh_qmat *m, float *d_out, void *stream) {
    int rc;
    if ((rc = check_qmat(m))) return rc;
    hipError_t e = jh::launch_dequant(m->type, m->d_raw, m->rows, m->cols, d_out, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail("dequant launch", e);
    return ok();
}

int jh_quantize_dev(int type, const float *d_src, int64_t n, void *d_dst, void *stream) {
    int qk, bb;
    if (!type_geometry(type, &qk, &bb)) return fail(JH_EUNSUPPORTED, "Re-quantisation not implemented for GGML type %d", type);
    if (n < 0 || n % qk) return fail(JH_EINVAL, "n=%lld is not a multiple of the block size %d", (long long)n, qk);
    hipError_t e = jh::launch_quantize(type, d_src, n, (uint8_t *)d_dst, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail("quantize launch", e);
    return ok();
}

// ---- the rest of the decode step

int jh_rmsnorm_dev(const float *x, const float *res, const float *w, int n, float eps, float *x_out, float *out,
                   void *stream) {
    if (n < 1 || n > (1 << 20)) return fail(JH_EINVAL, "n=%d outside [1, 2^20]", n);
    if (!x || !w || !out) return fail(JH_EINVAL, "x, w and out must not be null");
    if (out == x || (x_out && out == x_out)) return fail(JH_EINVAL, "out must not alias x or x_out");
    hipError_t e = jh::launch_rmsnorm(x, res, w, n, 1, eps, x_out, out, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail("rmsnorm launch", e);
    return ok();
}

int jh_rmsnorm_rows_dev(const float *x, const float *res, const float *w, int n, int rows, float eps, float *x_out,
                        float *out, void *stream) {
    if (n < 1 || n > (1 << 20)) return fail(JH_EINVAL, "n=%d outside [1, 2^20]", n);
    if (rows < 0 || rows > 65535) return fail(JH_EINVAL, "rows=%d outside [0, 65535]", rows);
    if (rows == 0) return ok();
    if (!x || !w || !out) return fail(JH_EINVAL, "x, w and out must not be null");
    if (out == x || (x_out && out == x_out)) return fail(JH_EINVAL, "out must not alias x or x_out");
    hipError_t e = jh::launch_rmsnorm(x, res, w, n, rows, eps, x_out, out, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail("rmsnorm launch", e);
    return ok();
}

static int check_heads(int n_heads, int n_kv_heads, int head_dim, int max_seq) {
    if (n_heads < 1 || n_kv_heads < 1 || n_heads % n_kv_heads)
        return fail(JH_EINVAL, "n_heads=%d must be a positive multiple of n_kv_heads=%d", n_heads, n_kv_heads);
    if (head_dim < 2 || head_dim % 2 || head_dim > 256)
        return fail(JH_EINVAL, "head_dim=%d must be even and in [2, 256]", head_dim);
    if (max_seq < 1 || max_seq > 32768) return fail(JH_EINVAL, "max_seq=%d outside [1, 32768]", max_seq);
    return JH_OK;
}

int jh_rope_kv_dev(float *q, const float *k, const float *v, int n_heads, int n_kv_heads, int head_dim,
                   const int *d_pos, int max_seq, float theta, float *k_cache, float *v_cache, void *stream) {
    int rc;
    if ((rc = check_heads(n_heads, n_kv_heads, head_dim, max_seq))) return rc;
    if (!q || !k || !v || !d_pos || !k_cache || !v_cache) return fail(JH_EINVAL, "pointers must not be null");
    hipError_t e = jh::launch_rope_kv(q, k, v, n_heads, n_kv_heads, head_dim, d_pos, max_seq, theta, k_cache, v_cache,
                                      (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail("rope_kv launch", e);
    return ok();
}

static int attention_common(const float *q, const float *k_new, const float *v_new, float *k_cache, float *v_cache,
                            int n_heads, int n_kv_heads, int head_dim, const int *d_pos, int max_seq, float theta,
                            bool fused, float *out, void *stream) {
    int rc;
    if ((rc = check_heads(n_heads, n_kv_heads, head_dim, max_seq))) return rc;
    if (!q || !k_cache || !v_cache || !d_pos || !out || (fused && (!k_new || !v_new)))
        return fail(JH_EINVAL, "pointers must not be null");
    int dev = 0;
    JH_HIP("hipGetDevice", hipGetDevice(&dev));
    void *ws = nullptr;
    if ((rc = stream_workspace(dev, (hipStream_t)stream, jh::attention_workspace_bytes(n_heads, head_dim, max_seq, 1),
                               &ws)))
        return rc;
    hipError_t e = jh::launch_attention(q, k_new, v_new, k_cache, v_cache, n_heads, n_kv_heads, head_dim, d_pos,
                                        max_seq, theta, fused, out, ws, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail("attention launch", e);
    return ok();
}

int jh_rope_attention_batched_dev(const float *q, const float *k, const float *v, int batch, int n_heads,
                                  int n_kv_heads, int head_dim, const int *d_pos, const int *d_slot, int n_slots,
                                  int max_seq, float theta, float *k_cache, float *v_cache, float *out, void *stream) {
    int rc;
    if ((rc = check_heads(n_heads, n_kv_heads, head_dim, max_seq))) return rc;
    if (batch < 0 || batch > 65535) return fail(JH_EINVAL, "batch=%d outside [0, 65535]", batch);
    if (n_slots < 1) return fail(JH_EINVAL, "n_slots=%d must be >= 1", n_slots);
    if (batch == 0) return ok();
    if (!q || !k || !v || !d_pos || !d_slot || !k_cache || !v_cache || !out)
        return fail(JH_EINVAL, "pointers must not be null");
    int dev = 0;
    JH_HIP("hipGetDevice", hipGetDevice(&dev));
    void *ws = nullptr;
    if ((rc = stream_workspace(dev, (hipStream_t)stream,
                               jh::attention_workspace_bytes(n_heads, head_dim, max_seq, batch), &ws)))
        return rc;
    hipError_t e = jh::launch_attention(q, k, v, k_cache, v_cache, n_heads, n_kv_heads, head_dim, d_pos, max_seq, theta,
                                        true, out, ws, (hipStream_t)stream, batch, d_slot, n_slots);
    if (e != hipSuccess) return hip_fail("attention launch", e);
    return ok();
}

// JUNO_ATTN_FUSE=1 moves attention's combine into the output projection's
// input conversion.  Not the default: every workgroup of the GEMV then reads all
// of the chunk partials (8B, position 511: 266 KB per CU against 37 KB of
// weights), and the projection takes the staged kernel; measured on MI355X, the
// 8B decode step went 2.071 -> 2.180 ms and the TinyLlama one 0.857 -> 0.936 ms.
static bool attn_fuse_wanted() {
    static const bool on = [] {
        const char *v = getenv("JUNO_ATTN_FUSE");
        return v && v[0] == '1';
    }();
    return on;
}

int jh_rope_attention_qmatvec_dev(const float *q, const float *k, const float *v, int n_heads, int n_kv_heads,
                                  int head_dim, const int *d_pos, int max_seq, float theta, float *k_cache,
                                  float *v_cache, const jh_qmat *wo, float *d_att, float *d_y, void *stream) {
    int rc;
    if ((rc = check_heads(n_heads, n_kv_heads, head_dim, max_seq))) return rc;
    if ((rc = check_qmat(wo))) return rc;
    if (!q || !k || !v || !d_pos || !k_cache || !v_cache || !d_att || !d_y)
        return fail(JH_EINVAL, "pointers must not be null");
    if ((long long)wo->cols != (long long)n_heads * head_dim)
        return fail(JH_EINVAL, "wo has %d columns, attention gives n_heads * head_dim = %lld", wo->cols,
                    (long long)n_heads * head_dim);
    {  // y is written while att is read (and, fused, while att is written)
        const uintptr_t a0 = reinterpret_cast<uintptr_t>(d_att), a1 = a0 + sizeof(float) * (size_t)wo->cols;
        const uintptr_t y0 = reinterpret_cast<uintptr_t>(d_y), y1 = y0 + sizeof(float) * (size_t)wo->rows;
        if (a0 < y1 && y0 < a1) return fail(JH_EINVAL, "att and y must not overlap");
    }
    int dev = 0;
    JH_HIP("hipGetDevice", hipGetDevice(&dev));
    void *ws = nullptr;
    if ((rc = stream_workspace(dev, (hipStream_t)stream, jh::attention_workspace_bytes(n_heads, head_dim, max_seq, 1),
                               &ws)))
        return rc;
    hipStream_t s = (hipStream_t)stream;
    int tc = 0, nch = 0;
    jh::attention_chunking(n_heads, n_kv_heads, head_dim, max_seq, 1, &tc, &nch);
    jh::GemvArgs a;
    a.type = wo->type;
    a.w = wo->d_raw;
    a.pitch = wo->pitch;
    a.cols = wo->cols;
    a.row_start = 0;
    a.row_end = wo->rows;
    a.batch = 1;
    a.x = nullptr;
    a.ldx = wo->cols;
    a.y = d_y;
    a.ldy = wo->rows;
    const jh::CombineSpec cs{static_cast<const float *>(ws), d_pos, head_dim, tc, max_seq, nch, d_att};
    const bool fuse = wo->type != JH_TYPE_F32 && gemv_path() != 1 && attn_fuse_wanted() && wo->rows > 0 &&
                      jh::launch_gemv_staged_combine(a, cs, s, true) == hipSuccess;
    hipError_t e = jh::launch_attention(q, k, v, k_cache, v_cache, n_heads, n_kv_heads, head_dim, d_pos, max_seq, theta,
                                        true, d_att, ws, s, 1, nullptr, 1, !fuse);
    if (e != hipSuccess) return hip_fail("attention launch", e);
    if (fuse) {
        const MatVecRange range(backend_label(wo->type), wo->rows, wo->cols, 1);
        e = jh::launch_gemv_staged_combine(a, cs, s);
        if (e != hipSuccess) return hip_fail("gemv_staged (attention combine) launch", e);
        return ok();
    }
    return jh_qmatvec_group_dev(1, &wo, (const float *const *)&d_att, &d_y, stream);
}

int jh_attention_dev(const float *q, const float *k_cache, const float *v_cache, int n_heads, int n_kv_heads,
                     int head_dim, const int *d_pos, int max_seq, float *out, void *stream) {
    return attention_common(q, nullptr, nullptr, const_cast<float *>(k_cache), const_cast<float *>(v_cache), n_heads,
                            n_kv_heads, head_dim, d_pos, max_seq, 0.f, false, out, stream);
}

int jh_rope_attention_dev(const float *q, const float *k, const float *v, int n_heads, int n_kv_heads, int head_dim,
                          const int *d_pos, int max_seq, float theta, float *k_cache, float *v_cache, float *out,
                          void *stream) {
    return attention_common(q, k, v, k_cache, v_cache, n_heads, n_kv_heads, head_dim, d_pos, max_seq, theta, true, out,
                            stream);
}

int jh_silu_mul_dev(const float *gate, const float *up, int n, float *out, void *stream) {
    if (n < 0) return fail(JH_EINVAL, "n=%d must be >= 0", n);
    if (n == 0) return ok();
    if (!gate || !up || !out) return fail(JH_EINVAL, "pointers must not be null");
    hipError_t e = jh::launch_silu_mul(gate, up, n, out, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail("silu_mul launch", e);
    return ok();
}

int jh_add_rows_dev(float *d_y, const float *d_bias, int n, int rows, void *stream) {
    if (n < 0 || rows < 0 || rows > 65535) return fail(JH_EINVAL, "n=%d and rows=%d must be >= 0 (rows <= 65535)", n, rows);
    if (n == 0 || rows == 0) return ok();
    if (!d_y || !d_bias) return fail(JH_EINVAL, "pointers must not be null");
    hipError_t e = jh::launch_add_rows(d_y, d_bias, n, rows, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail("add_rows launch", e);
    return ok();
}

int jh_lora_apply_dev(const float *d_a, const float *d_b, int rank, int in_dim, int out_dim, float scale,
                      const float *d_x, int batch, float *d_y, void *stream) {
    if (rank < 1 || rank > 4096) return fail(JH_EINVAL, "rank=%d outside [1, 4096]", rank);
    if (in_dim < 1 || out_dim < 1) return fail(JH_EINVAL, "inDim=%d and outDim=%d must be >= 1", in_dim, out_dim);
    if (batch < 0 || batch > 65535) return fail(JH_EINVAL, "batch=%d outside [0, 65535]", batch);
    if (batch == 0) return ok();
    if (!d_a || !d_b || !d_x || !d_y) return fail(JH_EINVAL, "pointers must not be null");
    int dev = 0, rc;
    JH_HIP("hipGetDevice", hipGetDevice(&dev));
    void *ws = nullptr;
    if ((rc = stream_workspace(dev, (hipStream_t)stream, (size_t)batch * rank * sizeof(float), &ws))) return rc;
    hipError_t e = jh::launch_lora(d_a, d_b, rank, in_dim, out_dim, scale, d_x, batch, d_y, static_cast<float *>(ws),
                                   (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail("lora launch", e);
    return ok();
}

int jh_pos_increment_dev(int *d_pos, int delta, void *stream) {
    if (!d_pos) return fail(JH_EINVAL, "d_pos must not be null");
    hipError_t e = jh::launch_pos_increment(d_pos, delta, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail("pos_increment launch", e);
    return ok();
}

int jh_embed_dev(const jh_qmat *m, const int *d_token, float *d_out, void *stream) {
    if (!m || !d_token || !d_out) return fail(JH_EINVAL, "matrix, token and out must not be null");
    if (m->rows <= 0) return fail(JH_EINVAL, "embedding matrix has no rows");
    int rc = set_device(m->ctx->device);
    if (rc) return rc;
    hipError_t e = jh::launch_dequant_row(m->type, m->d_raw, m->rows, m->cols, m->pitch, d_token, 1, d_out,
                                          (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail("embedding launch", e);
    return ok();
}

int jh_embed_rows_dev(const jh_qmat *m, const int *d_tokens, int n, float *d_out, void *stream) {
    if (n < 0 || n > 65535) return fail(JH_EINVAL, "n=%d outside [0, 65535]", n);
    if (n == 0) return ok();
    if (!m || !d_tokens || !d_out) return fail(JH_EINVAL, "matrix, tokens and out must not be null");
    if (m->rows <= 0) return fail(JH_EINVAL, "embedding matrix has no rows");
    int rc = set_device(m->ctx->device);
    if (rc) return rc;
    hipError_t e = jh::launch_dequant_row(m->type, m->d_raw, m->rows, m->cols, m->pitch, d_tokens, n, d_out,
                                          (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail("embedding launch", e);
    return ok();
}

int jh_gguf_upload(jh_ctx *ctx, const jh_gguf *g, int64_t index, jh_qmat **out) {
    if (!ctx || !g || !out) return fail(JH_EINVAL, "ctx, gguf and out must not be null");
    int64_t nbytes = 0, rows = 0, cols = 0;
    int type = 0;
    int rc = jh_gguf_stream_to_device(g, index, nullptr, &nbytes, &type, &rows, &cols);
    if (rc) return rc;
    if (rows > INT32_MAX || cols > INT32_MAX)
        return fail(JH_EINVAL, "tensor %lld is too large for a matrix: rows=%lld cols=%lld", (long long)index,
                    (long long)rows, (long long)cols);
    jh_qmat *m;
    rc = qmat_alloc(ctx, type, (int)rows, (int)cols, &m);
    if (rc) return rc;
    if ((int64_t)m->nbytes != nbytes) {
        jh_qmat_free(m);
        return fail(JH_EINVAL, "tensor %lld: %lld bytes on file != %zu for rows=%lld cols=%lld", (long long)index,
                    (long long)nbytes, m->nbytes, (long long)rows, (long long)cols);
    }
    rc = jh_gguf_stream_to_device(g, index, m->d_raw, nullptr, nullptr, nullptr, nullptr);
    if (rc) {
        std::string err = g_last_error;
        jh_qmat_free(m);
        g_last_error = err;
        return rc;
    }
    *out = m;
    return ok();
}

}  // extern "C"
