// The C ABI of libonegpu_hip.so (include/onegpu_hip.h): contexts, buffers, timing, and the validated entry points of
// the int8 path. Validation restates the reference's host-side checks (Int8Gemm.Prepare / CheckRange / CheckVector,
// Int8Gemm.cs:393-501; Check.Range / RangeBytes, KernelSupport.cs:75-110) in terms of byte sizes, so a caller that
// skipped them still cannot make a kernel read or write outside its buffers.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "og_internal.hpp"

struct og_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    og::Workspace ws{};
    // Workspaces replaced by larger ones: work recorded earlier (or captured into a graph) may still name them, so
    // they are freed only by og_destroy.
    std::vector<void *> retired;
    // The one-launch few-rows kernel's words (one a column slab, zero between launches) and the flag it raises in
    // host memory if a slab's tiles did not share an XCD or its parts were never all counted; xcd_local: og_init's
    // probe saw workgroup ids dealt round-robin to the XCDs, so that kernel may run.
    unsigned long long *xcd_words = nullptr;
    uint64_t xcd_word_count = 0;
    uint32_t *xcd_flag = nullptr;
    bool xcd_local = false;
    // Polls of a slab's count before that kernel's finishing tile gives up (og_test_set_spin_limit changes it).
    uint32_t spin_limit = og::kGemvSpinLimit;
    // og_int8_gemm_noalloc's fixed scratch on this device (og::noalloc_scratch_setup).
    uint8_t *noalloc_scratch = nullptr;
    std::string error;
    std::string argument;
    const char *last_kernel = "";
    std::string name;
    uint32_t compute_units = 0;
    uint32_t lds_bytes = 0;
    uint64_t max_buffer = 0;
    // timing
    bool timing = false;
    int timing_max = 0;
    int timing_n = 0;
    std::vector<hipEvent_t> ev_start, ev_stop;
    std::vector<const char *> ev_name;
    hipEvent_t region_start = nullptr, region_stop = nullptr;
    bool region_open = false;
};

namespace {

thread_local std::string t_error;
thread_local std::string t_argument;

constexpr uint64_t kInitialPartialBytes = 32ull << 20;

int fail(og_ctx *ctx, int status, const char *argument, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (ctx) {
        ctx->error = buf;
        ctx->argument = argument ? argument : "";
    }
    t_error = buf;
    t_argument = argument ? argument : "";
    return status;
}

int ok(og_ctx *ctx)
{
    if (ctx) {
        ctx->error.clear();
        ctx->argument.clear();
    }
    return OG_OK;
}

int hip_status(og_ctx *ctx, hipError_t e, const char *what)
{
    if (e == hipSuccess) return OG_OK;
    int st = OG_ERR_LAUNCH_FAILED;
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) st = OG_ERR_OUT_OF_MEMORY;
    else if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) st = OG_ERR_NO_DEVICE;
    else if (e == hipErrorLaunchFailure || e == hipErrorIllegalAddress || e == hipErrorECCNotCorrectable) st = OG_ERR_DEVICE_LOST;
    return fail(ctx, st, nullptr, "%s: %s (%s)", what, hipGetErrorString(e), hipGetErrorName(e));
}

// Brackets one kernel launch with timing events when timing is on.
template <typename F>
int launch(og_ctx *ctx, const char *what, F &&f)
{
    const char *name = "";
    bool timed = ctx->timing && ctx->timing_n < ctx->timing_max;
    if (timed) (void)hipEventRecord(ctx->ev_start[ctx->timing_n], ctx->stream);
    hipError_t e = f(&name);
    ctx->last_kernel = name;
    if (timed) {
        (void)hipEventRecord(ctx->ev_stop[ctx->timing_n], ctx->stream);
        ctx->ev_name[ctx->timing_n] = name;
        ctx->timing_n++;
    }
    return hip_status(ctx, e, what);
}

bool fits(uint64_t offset_bytes, uint64_t extent_bytes, const og_buffer &b)
{
    return offset_bytes <= b.bytes && extent_bytes <= b.bytes - offset_bytes;
}

// A workspace must grow: refused while the stream is being captured into a graph (the allocation would not be part
// of the graph, and a replay must not find its memory freed); otherwise allowed, and the caller retires the old one.
int growth_allowed(og_ctx *ctx, const char *what)
{
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(ctx->stream, &cs);
    if (e != hipSuccess) return hip_status(ctx, e, what);
    if (cs != hipStreamCaptureStatusNone)
        return fail(ctx, OG_ERR_INVALID_ARG, "workspace",
                    "%s must grow while the stream is being captured: run one product of this size before capturing", what);
    return OG_OK;
}

int ensure_partials(og_ctx *ctx, uint64_t bytes)
{
    if (bytes <= ctx->ws.partial_bytes) return OG_OK;
    int st = growth_allowed(ctx, "the partial-sum workspace");
    if (st != OG_OK) return st;
    // Grow geometrically. Work already recorded may still use the old region, and a graph captured earlier may name
    // it, so it is kept until og_destroy rather than freed.
    uint64_t size = ctx->ws.partial_bytes * 2 > bytes ? ctx->ws.partial_bytes * 2 : bytes;
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, size);
    if (e != hipSuccess) return hip_status(ctx, e, "workspace");
    if (ctx->ws.partials) ctx->retired.push_back(ctx->ws.partials);
    ctx->ws.partials = static_cast<int32_t *>(p);
    ctx->ws.partial_bytes = size;
    return OG_OK;
}

// The one-launch few-rows kernel's words: zero when allocated, and every launch leaves them zero.
int ensure_xcd_words(og_ctx *ctx, uint64_t words)
{
    if (words <= ctx->xcd_word_count) return OG_OK;
    int st = growth_allowed(ctx, "the few-rows count words");
    if (st != OG_OK) return st;
    uint64_t n = ctx->xcd_word_count * 2 > words ? ctx->xcd_word_count * 2 : words;
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, n * 8);
    if (e == hipSuccess) e = og::launch_fill_bytes(p, 0, n * 8, ctx->stream);
    if (e != hipSuccess) {
        if (p) (void)hipFree(p);
        return hip_status(ctx, e, "workspace");
    }
    if (ctx->xcd_words) ctx->retired.push_back(ctx->xcd_words);
    ctx->xcd_words = static_cast<unsigned long long *>(p);
    ctx->xcd_word_count = n;
    return OG_OK;
}

// Whether this device deals workgroup ids round-robin to its XCDs (id x on XCD (x + c) % 8 for one c a launch), which
// the one-launch few-rows kernel needs: all tiles of a column slab have ids equal modulo 8. Two probe launches of
// 4096 workgroups record where each ran.
bool probe_xcd_mapping(og_ctx *ctx)
{
    constexpr uint32_t kGroups = 4096;
    uint32_t *d = nullptr;
    std::vector<uint32_t> h(kGroups);
    bool good = hipMalloc(&d, kGroups * 4) == hipSuccess;
    for (int rep = 0; good && rep < 2; rep++) {
        good = og::launch_xcc_probe(d, kGroups, ctx->stream) == hipSuccess &&
               hipMemcpyAsync(h.data(), d, kGroups * 4, hipMemcpyDeviceToHost, ctx->stream) == hipSuccess &&
               hipStreamSynchronize(ctx->stream) == hipSuccess;
        for (uint32_t x = 0; good && x < kGroups; x++) good = h[x] == ((h[0] + x) & 7u);
    }
    if (d) (void)hipFree(d);
    return good;
}

}  // namespace

extern "C" {

const char *og_version(void) { return "onegpu-hip 0.1 (gfx950)"; }

const char *og_last_error(og_ctx *ctx) { return ctx ? ctx->error.c_str() : t_error.c_str(); }

const char *og_last_error_argument(og_ctx *ctx) { return ctx ? ctx->argument.c_str() : t_argument.c_str(); }

const char *og_last_kernel(og_ctx *ctx) { return ctx ? ctx->last_kernel : ""; }

int og_device_count(int *count)
{
    if (!count) return fail(nullptr, OG_ERR_INVALID_ARG, "count", "null pointer");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    *count = e == hipSuccess ? n : 0;
    return OG_OK;
}

int og_init(int device_ordinal, og_ctx **out)
{
    if (!out) return fail(nullptr, OG_ERR_INVALID_ARG, "out", "null pointer");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(nullptr, OG_ERR_NO_DEVICE, nullptr, "no HIP device");
    if (device_ordinal < 0 || device_ordinal >= n)
        return fail(nullptr, OG_ERR_INVALID_ARG, "device_ordinal", "device %d of %d", device_ordinal, n);
    og_ctx *ctx = new og_ctx();
    ctx->device = device_ordinal;
    hipError_t e = hipSetDevice(device_ordinal);
    hipDeviceProp_t prop{};
    if (e == hipSuccess) e = hipGetDeviceProperties(&prop, device_ordinal);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMalloc(&ctx->ws.partials, kInitialPartialBytes);
    if (e == hipSuccess) {
        ctx->ws.partial_bytes = kInitialPartialBytes;
        void *p = nullptr;
        // the dynamic quantizer's per-workgroup ranges (2 * kDqMaxGroups floats)
        size_t bytes = 2 * og::kDqMaxGroups * sizeof(float);
        e = hipMalloc(&p, bytes);
        if (e == hipSuccess) {
            ctx->ws.dq_ranges = static_cast<float *>(p);
        } else if (p) {
            (void)hipFree(p);
        }
    }
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void **>(&ctx->xcd_flag), sizeof(uint32_t), hipHostMallocDefault);
    if (e == hipSuccess) {
        *ctx->xcd_flag = 0;
        ctx->xcd_local = probe_xcd_mapping(ctx);
        e = hipGetLastError();
    }
    if (e == hipSuccess && ensure_xcd_words(ctx, 4096) != OG_OK) e = hipErrorOutOfMemory;
    if (e == hipSuccess) {
        void *p = nullptr;
        e = og::noalloc_scratch_setup(device_ordinal, ctx->stream, &p);
        ctx->noalloc_scratch = static_cast<uint8_t *>(p);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        int st = hip_status(nullptr, e, "og_init");
        og_destroy(ctx);
        return st;
    }
    ctx->name = prop.name;
    if (prop.gcnArchName[0]) ctx->name += std::string(" (") + prop.gcnArchName + ")";
    ctx->compute_units = (uint32_t)prop.multiProcessorCount;
    ctx->lds_bytes = (uint32_t)prop.sharedMemPerBlock;
    ctx->max_buffer = (uint64_t)prop.totalGlobalMem;
    *out = ctx;
    return OG_OK;
}

int og_destroy(og_ctx *ctx)
{
    if (!ctx) return OG_OK;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (auto e : ctx->ev_start) (void)hipEventDestroy(e);
    for (auto e : ctx->ev_stop) (void)hipEventDestroy(e);
    if (ctx->region_start) (void)hipEventDestroy(ctx->region_start);
    if (ctx->region_stop) (void)hipEventDestroy(ctx->region_stop);
    if (ctx->ws.partials) (void)hipFree(ctx->ws.partials);
    if (ctx->ws.dq_ranges) (void)hipFree(ctx->ws.dq_ranges);
    if (ctx->xcd_words) (void)hipFree(ctx->xcd_words);
    for (void *p : ctx->retired) (void)hipFree(p);
    if (ctx->xcd_flag) (void)hipHostFree(ctx->xcd_flag);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return OG_OK;
}

int og_device_name(og_ctx *ctx, char *buf, size_t len)
{
    if (!ctx || !buf || len == 0) return fail(ctx, OG_ERR_INVALID_ARG, "buf", "null context or buffer");
    snprintf(buf, len, "%s", ctx->name.c_str());
    return ok(ctx);
}

int og_device_limits(og_ctx *ctx, uint64_t *max_buffer_bytes, uint32_t *compute_units, uint32_t *lds_bytes)
{
    if (!ctx) return fail(ctx, OG_ERR_INVALID_ARG, "ctx", "null context");
    if (max_buffer_bytes) *max_buffer_bytes = ctx->max_buffer;
    if (compute_units) *compute_units = ctx->compute_units;
    if (lds_bytes) *lds_bytes = ctx->lds_bytes;
    return ok(ctx);
}

int og_stream(og_ctx *ctx, void **hip_stream)
{
    if (!ctx || !hip_stream) return fail(ctx, OG_ERR_INVALID_ARG, "hip_stream", "null context or pointer");
    *hip_stream = ctx->stream;
    return ok(ctx);
}

int og_sync(og_ctx *ctx)
{
    if (!ctx) return fail(ctx, OG_ERR_INVALID_ARG, "ctx", "null context");
    (void)hipSetDevice(ctx->device);
    int st = hip_status(ctx, hipStreamSynchronize(ctx->stream), "og_sync");
    if (st == OG_OK && ctx->xcd_flag && __atomic_load_n(ctx->xcd_flag, __ATOMIC_ACQUIRE) != 0) {
        // A one-launch few-rows product found a column slab's tiles on different XCDs (flag 1: its sums may be
        // wrong), gave up waiting for a slab's parts (flag 2: that slab's columns of C were not written), or found
        // the words poisoned by such a failure (flag 3: not run). Tiles may have counted into the words after the
        // failure, so the words this context's products use are cleared, the device's fixed ones too (a product of
        // og_int8_gemm_noalloc may have been the one that failed), and the context stops using that kernel.
        const uint32_t why = *ctx->xcd_flag;
        ctx->xcd_local = false;
        hipError_t e = hipSuccess;
        if (ctx->xcd_words) e = og::launch_fill_bytes(ctx->xcd_words, 0, ctx->xcd_word_count * 8, ctx->stream);
        if (e == hipSuccess && ctx->noalloc_scratch)
            e = og::launch_fill_bytes(ctx->noalloc_scratch, 0, og::kNoAllocWordBytes, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        __atomic_store_n(ctx->xcd_flag, 0u, __ATOMIC_RELEASE);
        if (e != hipSuccess) return hip_status(ctx, e, "og_sync");
        return fail(ctx, OG_ERR_LAUNCH_FAILED, nullptr,
                    why == 2   ? "og_sync: a one-launch few-rows product timed out waiting for a column slab's parts; "
                                 "its output is incomplete and the two-launch form is used from now on"
                    : why == 3 ? "og_sync: a one-launch few-rows product found its count words left by an earlier "
                                 "failed product and did not run; the two-launch form is used from now on"
                               : "og_sync: a one-launch few-rows product ran a column slab's tiles on different XCDs; "
                                 "its output may be wrong and the two-launch form is used from now on");
    }
    return st == OG_OK ? ok(ctx) : st;
}

int og_alloc(og_ctx *ctx, uint64_t bytes, void **dptr)
{
    if (!ctx || !dptr) return fail(ctx, OG_ERR_INVALID_ARG, "dptr", "null context or pointer");
    *dptr = nullptr;
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipMalloc(dptr, bytes ? bytes : 4);
    if (e != hipSuccess) return fail(ctx, OG_ERR_OUT_OF_MEMORY, "bytes", "hipMalloc of %llu bytes: %s", (unsigned long long)bytes, hipGetErrorString(e));
    return ok(ctx);
}

int og_free(og_ctx *ctx, void *dptr)
{
    if (!ctx) return fail(ctx, OG_ERR_INVALID_ARG, "ctx", "null context");
    if (!dptr) return ok(ctx);
    (void)hipSetDevice(ctx->device);
    // The buffer may still be named by recorded work: wait for the stream before releasing it.
    (void)hipStreamSynchronize(ctx->stream);
    int st = hip_status(ctx, hipFree(dptr), "og_free");
    return st == OG_OK ? ok(ctx) : st;
}

static int copy(og_ctx *ctx, void *dst, const void *src, uint64_t bytes, hipMemcpyKind kind, bool wait)
{
    if (!ctx) return fail(ctx, OG_ERR_INVALID_ARG, "ctx", "null context");
    if (bytes == 0) return ok(ctx);
    if (!dst || !src) return fail(ctx, OG_ERR_INVALID_ARG, dst ? "src" : "dst", "null pointer");
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, ctx->stream);
    if (e == hipSuccess && wait) e = hipStreamSynchronize(ctx->stream);
    int st = hip_status(ctx, e, "og_memcpy");
    return st == OG_OK ? ok(ctx) : st;
}

int og_memcpy_h2d(og_ctx *ctx, void *dst, const void *src, uint64_t bytes) { return copy(ctx, dst, src, bytes, hipMemcpyHostToDevice, true); }
int og_memcpy_d2h(og_ctx *ctx, void *dst, const void *src, uint64_t bytes) { return copy(ctx, dst, src, bytes, hipMemcpyDeviceToHost, true); }
int og_memcpy_d2d(og_ctx *ctx, void *dst, const void *src, uint64_t bytes) { return copy(ctx, dst, src, bytes, hipMemcpyDeviceToDevice, false); }

int og_fill_bytes(og_ctx *ctx, void *dst, uint8_t value, uint64_t bytes)
{
    if (!ctx) return fail(ctx, OG_ERR_INVALID_ARG, "ctx", "null context");
    if (bytes && !dst) return fail(ctx, OG_ERR_INVALID_ARG, "dst", "null pointer");
    (void)hipSetDevice(ctx->device);
    int st = launch(ctx, "og_fill_bytes", [&](const char **k) { *k = "fill-bytes"; return og::launch_fill_bytes(dst, value, bytes, ctx->stream); });
    return st == OG_OK ? ok(ctx) : st;
}

// ------------------------------------------------------------------ timing

int og_timing_begin(og_ctx *ctx, int max_dispatches)
{
    if (!ctx) return fail(ctx, OG_ERR_INVALID_ARG, "ctx", "null context");
    if (max_dispatches < 1) return fail(ctx, OG_ERR_INVALID_ARG, "max_dispatches", "must be at least 1, got %d", max_dispatches);
    (void)hipSetDevice(ctx->device);
    // Timing-only events: no system-scope fence (an L2 writeback and invalidate) when an event completes, so a pair
    // around a short dispatch measures the dispatch rather than the cache maintenance.
    constexpr unsigned kTimingEvent = hipEventDisableSystemFence;
    while ((int)ctx->ev_start.size() < max_dispatches) {
        hipEvent_t a, b;
        if (hipEventCreateWithFlags(&a, kTimingEvent) != hipSuccess) return fail(ctx, OG_ERR_OUT_OF_MEMORY, nullptr, "hipEventCreate");
        if (hipEventCreateWithFlags(&b, kTimingEvent) != hipSuccess) { (void)hipEventDestroy(a); return fail(ctx, OG_ERR_OUT_OF_MEMORY, nullptr, "hipEventCreate"); }
        ctx->ev_start.push_back(a);
        ctx->ev_stop.push_back(b);
        ctx->ev_name.push_back("");
    }
    ctx->timing = true;
    ctx->timing_max = max_dispatches;
    ctx->timing_n = 0;
    return ok(ctx);
}

int og_timing_end(og_ctx *ctx, int *dispatches)
{
    if (!ctx) return fail(ctx, OG_ERR_INVALID_ARG, "ctx", "null context");
    ctx->timing = false;
    if (dispatches) *dispatches = ctx->timing_n;
    return ok(ctx);
}

int og_timing_read(og_ctx *ctx, int index, float *ms, const char **kernel_name)
{
    if (!ctx) return fail(ctx, OG_ERR_INVALID_ARG, "ctx", "null context");
    if (index < 0 || index >= ctx->timing_n) return fail(ctx, OG_ERR_INVALID_ARG, "index", "%d outside the %d timed dispatches", index, ctx->timing_n);
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipEventSynchronize(ctx->ev_stop[index]);
    float t = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&t, ctx->ev_start[index], ctx->ev_stop[index]);
    if (e != hipSuccess) return hip_status(ctx, e, "og_timing_read");
    if (ms) *ms = t;
    if (kernel_name) *kernel_name = ctx->ev_name[index];
    return ok(ctx);
}

int og_timing_region_begin(og_ctx *ctx)
{
    if (!ctx) return fail(ctx, OG_ERR_INVALID_ARG, "ctx", "null context");
    (void)hipSetDevice(ctx->device);
    for (hipEvent_t *e : {&ctx->region_start, &ctx->region_stop})
        if (!*e && hipEventCreateWithFlags(e, hipEventDisableSystemFence) != hipSuccess)
            return fail(ctx, OG_ERR_OUT_OF_MEMORY, nullptr, "hipEventCreate");
    hipError_t e = hipEventRecord(ctx->region_start, ctx->stream);
    if (e != hipSuccess) return hip_status(ctx, e, "og_timing_region_begin");
    ctx->region_open = true;
    return ok(ctx);
}

int og_timing_region_end(og_ctx *ctx, float *ms)
{
    if (!ctx) return fail(ctx, OG_ERR_INVALID_ARG, "ctx", "null context");
    if (!ctx->region_open) return fail(ctx, OG_ERR_INVALID_ARG, "ctx", "og_timing_region_begin was not called");
    ctx->region_open = false;
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipEventRecord(ctx->region_stop, ctx->stream);
    if (e == hipSuccess) e = hipEventSynchronize(ctx->region_stop);
    float t = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&t, ctx->region_start, ctx->region_stop);
    if (e != hipSuccess) return hip_status(ctx, e, "og_timing_region_end");
    if (ms) *ms = t;
    return ok(ctx);
}

}  // extern "C"

// ------------------------------------------------------------------ Int8Gemm

namespace og {

GemmKernel choose_gemm_kernel(int32_t M, int32_t N, int32_t K, int32_t batch, uint32_t flags)
{
    (void)N;
    (void)batch;
    if (flags & OG_GEMM_PORTABLE) return GemmKernel::Portable;
    const bool trans_b = flags & OG_GEMM_TRANSPOSE_B;
    // Few rows against weights stored K x N: stream B once (the reference's row kernel regime, Int8Gemm.cs:562-563).
    if (!trans_b && M <= 16 && K > 0 && !(flags & OG_GEMM_NO_SKINNY)) {
        if (skinny_slices(M, N, K, batch) <= 1 && !(flags & OG_GEMM_NO_DIRECT)) return GemmKernel::SkinnyDirect;
        return GemmKernel::Skinny;
    }
    return GemmKernel::Tiled;
}

const char *gemm_kernel_name(GemmKernel k)
{
    switch (k) {
    case GemmKernel::Portable: return "portable-tile64x64x16";
    case GemmKernel::Skinny: return "mfma-i8-rows16-splitk";
    case GemmKernel::SkinnyDirect: return "mfma-i8-rows16-direct";
    case GemmKernel::RowTiles: return "mfma-i8-rows16-tiles";
    case GemmKernel::RowXcd: return "mfma-i8-rows16-xcd";
    default: return "mfma-i8-tile128x128x64";
    }
}

}  // namespace og

extern "C" {

static const uint32_t kKnownGemmFlags =
    0x7Fu | 0x380u | OG_GEMM_PORTABLE | OG_GEMM_NO_SKINNY | OG_GEMM_NO_DIRECT | OG_GEMM_LARGE_TILE | OG_GEMM_NO_STREAM |
    OG_GEMM_TWO_PASS;

// Checks the parameter block alone; returns OG_OK or the failing status (message and argument set).
// `requant`: the parameters of og_int8_gemm_requantized, whose Epi holds only the int bias and per-column bits.
static int check_gemm_params(og_ctx *ctx, const og_int8_gemm_params *p, uint32_t batch, bool requant = false)
{
    if (!p) return fail(ctx, OG_ERR_INVALID_ARG, "params", "null parameter block");
    const uint32_t imax = 0x7FFFFFFFu;
    if (p->M > imax) return fail(ctx, OG_ERR_INVALID_ARG, "M", "must not be negative, got %d", (int32_t)p->M);
    if (p->N > imax) return fail(ctx, OG_ERR_INVALID_ARG, "N", "must not be negative, got %d", (int32_t)p->N);
    if (p->K > imax) return fail(ctx, OG_ERR_INVALID_ARG, "K", "must not be negative, got %d", (int32_t)p->K);
    if (batch < 1 || batch > imax) return fail(ctx, OG_ERR_INVALID_ARG, "Batch", "must be at least 1, got %d", (int32_t)batch);
    if (p->Flags & ~kKnownGemmFlags) return fail(ctx, OG_ERR_INVALID_ARG, "Flags", "unknown flag bits 0x%x", p->Flags & ~kKnownGemmFlags);
    if ((p->Flags & OG_GEMM_ZA_PER_ROW) && !(p->Flags & OG_GEMM_ZA)) return fail(ctx, OG_ERR_INVALID_ARG, "Flags", "per-row zero point without a zero point");
    if ((p->Flags & OG_GEMM_ZB_PER_COL) && !(p->Flags & OG_GEMM_ZB)) return fail(ctx, OG_ERR_INVALID_ARG, "Flags", "per-column zero point without a zero point");
    if (requant) {
        if (p->Epi & ~(OG_EPI_INT_BIAS | OG_EPI_SCALE_PER_COL))
            return fail(ctx, OG_ERR_INVALID_ARG, "Epi", "a requantized product takes only the int bias and per-column multiplier bits, got 0x%x", p->Epi);
    } else {
        if (p->Epi & ~0xFu) return fail(ctx, OG_ERR_INVALID_ARG, "Epi", "unknown epilogue bits 0x%x", p->Epi & ~0xFu);
        if ((p->Epi & (OG_EPI_SCALE_PER_COL | OG_EPI_FLOAT_BIAS)) && !(p->Epi & OG_EPI_FLOAT))
            return fail(ctx, OG_ERR_INVALID_ARG, "Epi", "a scale or float bias needs the float result bit");
    }
    const bool trans_b = p->Flags & OG_GEMM_TRANSPOSE_B;
    const uint64_t lda = p->Lda ? p->Lda : (p->K ? p->K : 1);
    const uint64_t cols_b = trans_b ? p->K : p->N;
    const uint64_t ldb = p->Ldb ? p->Ldb : (cols_b ? cols_b : 1);
    if (lda > imax || lda < p->K) return fail(ctx, OG_ERR_INVALID_ARG, "Lda", "%llu is smaller than K = %u", (unsigned long long)lda, p->K);
    if (ldb > imax || ldb < cols_b) return fail(ctx, OG_ERR_INVALID_ARG, "Ldb", "%llu is smaller than the stored row length %llu", (unsigned long long)ldb, (unsigned long long)cols_b);
    if ((uint64_t)batch * p->M * p->N > imax) return fail(ctx, OG_ERR_INVALID_ARG, "Batch", "the result holds more elements than the kernels address");
    if (p->M > 0 && p->N > 0 && p->StrideC < (uint64_t)p->M * p->N && batch > 1)
        return fail(ctx, OG_ERR_INVALID_ARG, "StrideC", "%u is smaller than M * N", p->StrideC);
    return OG_OK;
}

int og_int8_gemm_kernel_name(const og_int8_gemm_params *p, uint32_t batch, char *buf, size_t len)
{
    if (!p || !buf || len == 0) return fail(nullptr, OG_ERR_INVALID_ARG, "params", "null pointer");
    const int32_t b = (int32_t)(batch ? batch : 1);
    og::GemmKernel k = og::choose_gemm_kernel((int32_t)p->M, (int32_t)p->N, (int32_t)p->K, b, p->Flags);
    const char *name = og::gemm_kernel_name(k);
    // The operands as og_int8_gemm would see them, with the offsets standing in for the addresses (buffers from
    // og_alloc are aligned), so that the alignment conditions of the kernels decide as they would.
    og::GemmArgs g{};
    g.A = reinterpret_cast<const uint8_t *>((uintptr_t)p->OffA);
    g.B = reinterpret_cast<const uint8_t *>((uintptr_t)p->OffB);
    g.M = (int32_t)p->M;
    g.N = (int32_t)p->N;
    g.K = (int32_t)p->K;
    g.batch = b;
    g.lda = (int32_t)(p->Lda ? p->Lda : (p->K ? p->K : 1));
    const uint32_t cols_b = (p->Flags & OG_GEMM_TRANSPOSE_B) ? p->K : p->N;
    g.ldb = (int32_t)(p->Ldb ? p->Ldb : (cols_b ? cols_b : 1));
    g.strideA = p->StrideA;
    g.strideB = p->StrideB;
    g.flags = p->Flags;
    // B as og_alloc leaves it: padded to a whole 32-bit word.
    g.b_bytes = (int64_t)(b - 1) * g.strideB + (int64_t)(g.K > 0 ? g.K - 1 : 0) * g.ldb + ((cols_b + 3) & ~3u);
    // The tiled family's name also says the kernel and tile (the same choice as launch_gemm_tiled).
    if (k == og::GemmKernel::Tiled) {
        const bool large = (p->Flags & OG_GEMM_LARGE_TILE) || og::tiled_uses_large(g.M, g.N, b);
        if (!og::tiled_fast_ok(g)) name = "mfma-i8-generic128x128x64";
        else if (og::direct_ok(g))
            name = large ? "mfma-i8-direct256x256x64"
                         : (og::direct_split(g) > 1 ? "mfma-i8-direct128x128x64-splitk" : "mfma-i8-direct128x128x64");
        else name = large ? "mfma-i8-tile256x256x64" : "mfma-i8-tile128x128x128";
    }
    // The few-rows products take the tiled kernel when the operands' rows are aligned.
    // In one launch unless asked for two (a context whose probe found no round-robin XCD mapping runs two as well:
    // og_last_kernel then names the kernel that ran).
    if ((k == og::GemmKernel::Skinny || k == og::GemmKernel::SkinnyDirect) && !(p->Flags & OG_GEMM_NO_STREAM) &&
        og::gemv_tiles_ok(g))
        name = og::gemm_kernel_name(!(p->Flags & OG_GEMM_TWO_PASS) && og::gemv_xcd_ok(g) ? og::GemmKernel::RowXcd
                                                                                         : og::GemmKernel::RowTiles);
    snprintf(buf, len, "%s", name);
    return OG_OK;
}

// Where a product's scratch comes from: the context's workspace, grown as needed, or (fixed) the device's array of
// og_int8_gemm_noalloc, which nothing grows: a product that needs more is refused.
struct ProductScratch {
    bool fixed = false;
    og::Workspace ws{};
    unsigned long long *words = nullptr;
    uint64_t word_count = 0;
};

static int scratch_for(og_ctx *ctx, ProductScratch &sc, uint64_t partial_bytes, uint64_t words)
{
    if (sc.fixed) {
        if (partial_bytes > sc.ws.partial_bytes || words > sc.word_count)
            return fail(ctx, OG_ERR_UNSUPPORTED, "scratch",
                        "the product needs %llu bytes of partial sums and %llu count words; the fixed scratch holds "
                        "%llu and %llu",
                        (unsigned long long)partial_bytes, (unsigned long long)words,
                        (unsigned long long)sc.ws.partial_bytes, (unsigned long long)sc.word_count);
        return OG_OK;
    }
    int st = ensure_partials(ctx, partial_bytes);
    if (st == OG_OK && words) st = ensure_xcd_words(ctx, words);
    sc.ws = ctx->ws;
    sc.words = ctx->xcd_words;
    sc.word_count = ctx->xcd_word_count;
    return st;
}

static int launch_product_kernel(og_ctx *ctx, const og::GemmArgs &g, og::GemmKernel k, int ks, ProductScratch &sc);

// Chooses the kernel for a validated product and launches it (two launches for the split few-rows forms), on ctx's
// stream with its device current. og_int8_gemm and the convolution's products come through here; `fixed` takes the
// scratch from og_int8_gemm_noalloc's array. A ranged float product (g.ranges set, C dense) sets *range_groups to the
// (min, max) pairs written at g.ranges: from the kernel's epilogue where it has one, else from a range pass over C.
static int launch_product(og_ctx *ctx, const og::GemmArgs &g_in, bool fixed = false, uint32_t *range_groups = nullptr)
{
    int st = OG_OK;
    og::GemmArgs g = g_in;
    ProductScratch sc;
    if (fixed) {
        sc.fixed = true;
        sc.words = reinterpret_cast<unsigned long long *>(ctx->noalloc_scratch);
        sc.word_count = og::kNoAllocWordBytes / 8;
        sc.ws.partials = reinterpret_cast<int32_t *>(ctx->noalloc_scratch + og::kNoAllocWordBytes);
        sc.ws.partial_bytes = og::kNoAllocScratchBytes - og::kNoAllocWordBytes;
        sc.ws.dq_ranges = ctx->ws.dq_ranges;
    }
    og::GemmKernel k = og::choose_gemm_kernel(g.M, g.N, g.K, g.batch, g.flags);
    if ((k == og::GemmKernel::Skinny || k == og::GemmKernel::SkinnyDirect) && !(g.flags & OG_GEMM_NO_STREAM) &&
        og::gemv_tiles_ok(g))
        // A raised flag that og_sync has not seen yet already rules the one-launch form out.
        k = ctx->xcd_local && __atomic_load_n(ctx->xcd_flag, __ATOMIC_ACQUIRE) == 0 && !(g.flags & OG_GEMM_TWO_PASS) &&
                    og::gemv_xcd_ok(g)
                ? og::GemmKernel::RowXcd
                : og::GemmKernel::RowTiles;
    // The split of a tiled product along K (the 128 x 128 direct kernel on grids under half the chip).
    const int ks = k == og::GemmKernel::Tiled && og::tiled_fast_ok(g) && og::direct_ok(g) &&
                           !og::tiled_uses_large(g.M, g.N, g.batch) && !(g.flags & OG_GEMM_LARGE_TILE)
                       ? og::direct_split(g)
                       : 1;
    // A ranged product: the pairs the chosen kernel's epilogue writes (0: it has no range epilogue, or more pairs than
    // the caller's buffer holds; the range pass over C runs after it instead).
    uint32_t epi_groups = 0;
    if (g.ranges) {
        if (k == og::GemmKernel::Tiled && og::tiled_fast_ok(g) && og::direct_ok(g))
            epi_groups = ks > 1 ? og::direct_split_range_groups(g)
                                : og::direct_range_groups(g, (g.flags & OG_GEMM_LARGE_TILE) ||
                                                                 og::tiled_uses_large(g.M, g.N, g.batch));
        else if (k == og::GemmKernel::RowXcd)
            epi_groups = og::gemv_xcd_range_groups(g);
        if (epi_groups > (uint32_t)og::kRangesMax) epi_groups = 0;
        if (epi_groups == 0) g.ranges = nullptr;
    }
    st = launch_product_kernel(ctx, g, k, ks, sc);
    if (st != OG_OK || !range_groups) return st;
    if (epi_groups) {
        *range_groups = epi_groups;
        return st;
    }
    // No range epilogue: a range pass over the dense float result.
    uint32_t groups = 0;
    const char *product = ctx->last_kernel;   // the product keeps its name
    st = launch(ctx, "og_int8_gemm", [&](const char **n) {
        return og::launch_range_pass(static_cast<const float *>(g.C), (uint32_t)((uint64_t)g.M * g.N * g.batch),
                                     g_in.ranges, ctx->stream, n, &groups);
    });
    ctx->last_kernel = product;
    *range_groups = groups;
    return st;
}

// Launches product kind k (ks > 1: the direct kernel split along K) with the scratch of `sc`.
static int launch_product_kernel(og_ctx *ctx, const og::GemmArgs &g, og::GemmKernel k, int ks, ProductScratch &sc)
{
    int st = OG_OK;
    switch (k) {
    case og::GemmKernel::Portable:
        st = launch(ctx, "og_int8_gemm", [&](const char **n) { return og::launch_gemm_portable(g, ctx->stream, n); });
        break;
    case og::GemmKernel::Tiled: {
        // A grid that fills under half the chip splits along K when it takes the 128 x 128 direct kernel.
        if (ks > 1) {
            st = scratch_for(ctx, sc, og::direct_split_workspace_bytes(g, ks), 0);
            if (st != OG_OK) return st;
            st = launch(ctx, "og_int8_gemm", [&](const char **n) { return og::launch_gemm_direct_split(g, sc.ws, ctx->stream, n, ks, 0); });
            if (st == OG_OK) {
                const char *product = ctx->last_kernel;   // named for the product, not the summing pass
                st = launch(ctx, "og_int8_gemm", [&](const char **n) { return og::launch_gemm_direct_split(g, sc.ws, ctx->stream, n, ks, 1); });
                ctx->last_kernel = product;
            }
            break;
        }
        st = launch(ctx, "og_int8_gemm", [&](const char **n) { return og::launch_gemm_tiled(g, ctx->stream, n); });
        break;
    }
    case og::GemmKernel::RowXcd:
        st = scratch_for(ctx, sc, og::gemv_xcd_workspace_bytes(g), og::gemv_xcd_words(g));
        if (st != OG_OK) return st;
        st = launch(ctx, "og_int8_gemm", [&](const char **n) {
            return og::launch_gemv_xcd(g, sc.ws.partials, sc.words, ctx->xcd_flag, ctx->spin_limit, ctx->stream, n);
        });
        break;
    case og::GemmKernel::RowTiles:
        st = scratch_for(ctx, sc, og::gemv_tiles_workspace_bytes(g), 0);
        if (st != OG_OK) return st;
        st = launch(ctx, "og_int8_gemm", [&](const char **n) { return og::launch_gemv_tiles(g, sc.ws, ctx->stream, n, 0); });
        if (st == OG_OK) {
            const char *product = ctx->last_kernel;   // the product is named for its tile kernel, not the summing pass
            st = launch(ctx, "og_int8_gemm", [&](const char **n) { return og::launch_gemv_tiles(g, sc.ws, ctx->stream, n, 1); });
            ctx->last_kernel = product;
        }
        break;
    case og::GemmKernel::SkinnyDirect:   // one slice: no partial sums
        st = launch(ctx, "og_int8_gemm", [&](const char **n) { return og::launch_gemm_skinny(g, ctx->ws, ctx->stream, n, 0); });
        break;
    case og::GemmKernel::Skinny:
        st = scratch_for(ctx, sc, og::skinny_workspace_bytes(g.M, g.N, g.K, g.batch), 0);
        if (st != OG_OK) return st;
        st = launch(ctx, "og_int8_gemm", [&](const char **n) { return og::launch_gemm_skinny(g, sc.ws, ctx->stream, n, 0); });
        if (st == OG_OK) {
            const char *product = ctx->last_kernel;   // named for the split-k kernel, not the reduction pass
            st = launch(ctx, "og_int8_gemm", [&](const char **n) { return og::launch_gemm_skinny(g, sc.ws, ctx->stream, n, 1); });
            ctx->last_kernel = product;
        }
        break;
    }
    return st;
}

// The output side of a requantized product (og_int8_gemm_requantized); absent for og_int8_gemm.
struct RequantOut {
    int32_t zero_point;
    bool is_signed;
};

// The range output of og_int8_gemm_float_ranged.
struct RangeOut {
    og_buffer ranges;
    uint32_t *groups;
};

// The activation scale of og_int8_gemm_float_scaled.
struct ActScale {
    og_buffer buf;
    uint32_t offset;
};

// og_int8_gemm and og_int8_gemm_requantized: validation, then the kernel choice and launch. With `rq`, C is the 8-bit
// output Y (OffC and StrideC in bytes) and `scale` the multiplier.
static int run_gemm(og_ctx *ctx, const og_int8_gemm_params *p, uint32_t batch, og_buffer A, og_buffer B, og_buffer C,
                    og_buffer ZA, og_buffer ZB, og_buffer bias, og_buffer scale, og_buffer fbias, const RequantOut *rq,
                    const ActScale *act = nullptr, bool fixed_scratch = false, const RangeOut *rout = nullptr)
{
    int st = check_gemm_params(ctx, p, batch, rq != nullptr);
    if (st != OG_OK) return st;
    if (rout) {
        if (!(p->Epi & OG_EPI_FLOAT) || rq) return fail(ctx, OG_ERR_INVALID_ARG, "Epi", "a ranged product needs the float result bit");
        if (!rout->groups) return fail(ctx, OG_ERR_INVALID_ARG, "groups", "null pointer");
        if (!rout->ranges.ptr || ((uintptr_t)rout->ranges.ptr & 7) || rout->ranges.bytes < 8ull * og::kRangesMax)
            return fail(ctx, OG_ERR_INVALID_ARG, "ranges", "the ranges need %d (min, max) pairs of float32, 8-byte aligned", og::kRangesMax);
        if (batch > 1 && p->StrideC != (uint64_t)p->M * p->N)
            return fail(ctx, OG_ERR_INVALID_ARG, "StrideC", "a ranged product's C is dense: StrideC must be M * N");
        if ((uint64_t)p->M * p->N * batch > 0x7FFFFFFFull)
            return fail(ctx, OG_ERR_INVALID_ARG, "c", "a ranged product's C holds more than 2147483647 elements");
        *rout->groups = 0;
    }
    if (act) {
        if (!(p->Epi & OG_EPI_FLOAT)) return fail(ctx, OG_ERR_INVALID_ARG, "Epi", "a scaled product needs the float result bit");
        if (!act->buf.ptr || ((uintptr_t)act->buf.ptr & 3)) return fail(ctx, OG_ERR_INVALID_ARG, "activationScale", "the activation scale is missing or misaligned");
        if (!fits((uint64_t)act->offset * 4, 4, act->buf)) return fail(ctx, OG_ERR_INVALID_ARG, "activationScale", "element %u reaches past the buffer of %llu", act->offset, (unsigned long long)(act->buf.bytes / 4));
    }
    const bool trans_b = p->Flags & OG_GEMM_TRANSPOSE_B;
    const uint64_t M = p->M, N = p->N, K = p->K;
    const uint64_t lda = p->Lda ? p->Lda : (K ? K : 1);
    const uint64_t rows_b = trans_b ? N : K, cols_b = trans_b ? K : N;
    const uint64_t ldb = p->Ldb ? p->Ldb : (cols_b ? cols_b : 1);
    const uint64_t stride_c = batch > 1 ? p->StrideC : M * N;
    // Operand ranges (Int8Gemm.CheckRange: the last byte an operand reaches lies inside its buffer).
    if (M > 0 && N > 0 && K > 0) {
        if (!A.ptr) return fail(ctx, OG_ERR_INVALID_ARG, "a", "A is missing");
        if (!B.ptr) return fail(ctx, OG_ERR_INVALID_ARG, "b", "B is missing");
        uint64_t last_a = p->OffA + (uint64_t)(batch - 1) * p->StrideA + (M - 1) * lda + (K - 1);
        if (last_a >= A.bytes) return fail(ctx, OG_ERR_INVALID_ARG, "OffsetA", "operand A reaches byte %llu but its buffer holds %llu", (unsigned long long)last_a, (unsigned long long)A.bytes);
        uint64_t last_b = p->OffB + (uint64_t)(batch - 1) * p->StrideB + (rows_b - 1) * ldb + (cols_b - 1);
        if (last_b >= B.bytes) return fail(ctx, OG_ERR_INVALID_ARG, "OffsetB", "operand B reaches byte %llu but its buffer holds %llu", (unsigned long long)last_b, (unsigned long long)B.bytes);
    }
    const uint64_t count_c = M * N ? (uint64_t)(batch - 1) * stride_c + M * N : 0;
    const uint64_t esize = rq ? 1 : 4;   // bytes per output element
    if (M > 0 && N > 0) {
        const char *name = rq ? "y" : "c";
        if (!C.ptr) return fail(ctx, OG_ERR_INVALID_ARG, name, "the output is missing");
        if (!rq && ((uintptr_t)C.ptr & 3) != 0) return fail(ctx, OG_ERR_INVALID_ARG, "c", "C is not 4-byte aligned");
        if (!fits((uint64_t)p->OffC * esize, count_c * esize, C)) return fail(ctx, OG_ERR_INVALID_ARG, name, "elements %u..%llu reach past the buffer of %llu", p->OffC, (unsigned long long)(p->OffC + count_c), (unsigned long long)(C.bytes / esize));
    }
    if (rq) {
        if (rq->zero_point < (rq->is_signed ? -128 : 0) || rq->zero_point > (rq->is_signed ? 127 : 255))
            return fail(ctx, OG_ERR_INVALID_ARG, "zeroPointY", "%d is outside the output type's range", rq->zero_point);
        const uint64_t n = (p->Epi & OG_EPI_SCALE_PER_COL) ? N : 1;
        if (!scale.ptr || ((uintptr_t)scale.ptr & 3)) return fail(ctx, OG_ERR_INVALID_ARG, "multiplier", "the multiplier is missing or misaligned");
        if (!fits((uint64_t)p->OffScale * 4, n * 4, scale)) return fail(ctx, OG_ERR_INVALID_ARG, "multiplier", "elements %u..%llu reach past the buffer of %llu", p->OffScale, (unsigned long long)(p->OffScale + n), (unsigned long long)(scale.bytes / 4));
    }
    const bool has_za = p->Flags & OG_GEMM_ZA, has_zb = p->Flags & OG_GEMM_ZB;
    if (has_za) {
        uint64_t n = (p->Flags & OG_GEMM_ZA_PER_ROW) ? M : 1;
        if (!ZA.ptr) return fail(ctx, OG_ERR_INVALID_ARG, "zpA", "the zero point of A is missing");
        if (!fits(p->OffZA, n, ZA)) return fail(ctx, OG_ERR_INVALID_ARG, "zpA", "elements %u..%llu reach past the buffer of %llu", p->OffZA, (unsigned long long)(p->OffZA + n), (unsigned long long)ZA.bytes);
    }
    if (has_zb) {
        uint64_t n = (p->Flags & OG_GEMM_ZB_PER_COL) ? N : 1;
        if (!ZB.ptr) return fail(ctx, OG_ERR_INVALID_ARG, "zpB", "the zero point of B is missing");
        if (!fits(p->OffZB, n, ZB)) return fail(ctx, OG_ERR_INVALID_ARG, "zpB", "elements %u..%llu reach past the buffer of %llu", p->OffZB, (unsigned long long)(p->OffZB + n), (unsigned long long)ZB.bytes);
    }
    if (p->Epi & OG_EPI_INT_BIAS) {
        if (!bias.ptr || ((uintptr_t)bias.ptr & 3)) return fail(ctx, OG_ERR_INVALID_ARG, "bias", "the int32 bias is missing or misaligned");
        if (!fits((uint64_t)p->OffBias * 4, N * 4, bias)) return fail(ctx, OG_ERR_INVALID_ARG, "bias", "elements %u..%llu reach past the buffer of %llu", p->OffBias, (unsigned long long)(p->OffBias + N), (unsigned long long)(bias.bytes / 4));
    }
    if (p->Epi & OG_EPI_FLOAT) {
        uint64_t n = (p->Epi & OG_EPI_SCALE_PER_COL) ? N : 1;
        if (!scale.ptr || ((uintptr_t)scale.ptr & 3)) return fail(ctx, OG_ERR_INVALID_ARG, "scale", "the scale is missing or misaligned");
        if (!fits((uint64_t)p->OffScale * 4, n * 4, scale)) return fail(ctx, OG_ERR_INVALID_ARG, "scale", "elements %u..%llu reach past the buffer of %llu", p->OffScale, (unsigned long long)(p->OffScale + n), (unsigned long long)(scale.bytes / 4));
    }
    if (p->Epi & OG_EPI_FLOAT_BIAS) {
        if (!fbias.ptr || ((uintptr_t)fbias.ptr & 3)) return fail(ctx, OG_ERR_INVALID_ARG, "floatBias", "the float bias is missing or misaligned");
        if (!fits((uint64_t)p->OffFBias * 4, N * 4, fbias)) return fail(ctx, OG_ERR_INVALID_ARG, "floatBias", "elements %u..%llu reach past the buffer of %llu", p->OffFBias, (unsigned long long)(p->OffFBias + N), (unsigned long long)(fbias.bytes / 4));
    }
    if (!ctx) return fail(ctx, OG_ERR_NO_DEVICE, "ctx", "no context: the arguments are valid but there is no device to run on");
    if (M == 0 || N == 0) return ok(ctx);

    og::GemmArgs g{};
    g.A = static_cast<const uint8_t *>(A.ptr) + p->OffA;
    g.B = static_cast<const uint8_t *>(B.ptr) + p->OffB;
    g.C = static_cast<uint8_t *>(C.ptr) + (uint64_t)p->OffC * esize;
    g.ZA = has_za ? static_cast<const uint8_t *>(ZA.ptr) + p->OffZA : nullptr;
    g.ZB = has_zb ? static_cast<const uint8_t *>(ZB.ptr) + p->OffZB : nullptr;
    g.bias = (p->Epi & OG_EPI_INT_BIAS) ? static_cast<const int32_t *>(bias.ptr) + p->OffBias : nullptr;
    g.scale = (p->Epi & OG_EPI_FLOAT) || rq ? static_cast<const float *>(scale.ptr) + p->OffScale : nullptr;
    g.fbias = (p->Epi & OG_EPI_FLOAT_BIAS) ? static_cast<const float *>(fbias.ptr) + p->OffFBias : nullptr;
    g.strideA = p->StrideA;
    g.strideB = p->StrideB;
    g.strideC = (int64_t)stride_c;
    g.b_bytes = B.ptr && B.bytes > p->OffB ? (int64_t)(B.bytes - p->OffB) : 0;
    g.M = (int32_t)M;
    g.N = (int32_t)N;
    g.K = (int32_t)K;
    g.batch = (int32_t)batch;
    g.lda = (int32_t)lda;
    g.ldb = (int32_t)ldb;
    g.flags = p->Flags;
    g.epi = p->Epi | (rq ? (og::EPI_REQUANT | (rq->is_signed ? 0u : og::EPI_REQUANT_U8)) : 0u) |
            (act ? og::EPI_SCALE_PRODUCT : 0u);
    g.act_scale = act ? static_cast<const float *>(act->buf.ptr) + act->offset : nullptr;
    g.zp_y = rq ? rq->zero_point : 0;
    g.ranges = rout ? static_cast<float *>(rout->ranges.ptr) : nullptr;

    (void)hipSetDevice(ctx->device);
    st = launch_product(ctx, g, fixed_scratch, rout ? rout->groups : nullptr);
    return st == OG_OK ? ok(ctx) : st;
}

int og_int8_gemm(og_ctx *ctx, const og_int8_gemm_params *p, uint32_t batch, og_buffer A, og_buffer B, og_buffer C,
                 og_buffer ZA, og_buffer ZB, og_buffer bias, og_buffer scale, og_buffer fbias)
{
    return run_gemm(ctx, p, batch, A, B, C, ZA, ZB, bias, scale, fbias, nullptr);
}

// og_int8_gemm with the device's fixed scratch array: nothing is allocated (no counterpart in the reference).
int og_int8_gemm_noalloc(og_ctx *ctx, const og_int8_gemm_params *p, uint32_t batch, og_buffer A, og_buffer B,
                         og_buffer C, og_buffer ZA, og_buffer ZB, og_buffer bias, og_buffer scale, og_buffer fbias)
{
    if (ctx && !ctx->noalloc_scratch) return fail(ctx, OG_ERR_UNSUPPORTED, "scratch", "the fixed scratch was not set up");
    return run_gemm(ctx, p, batch, A, B, C, ZA, ZB, bias, scale, fbias, nullptr, nullptr, true);
}

int og_int8_gemm_float_scaled(og_ctx *ctx, const og_int8_gemm_params *p, uint32_t batch, og_buffer A, og_buffer B,
                              og_buffer C, og_buffer ZA, og_buffer ZB, og_buffer bias, og_buffer act_scale,
                              uint32_t act_offset, og_buffer scale, og_buffer fbias)
{
    const ActScale act{act_scale, act_offset};
    return run_gemm(ctx, p, batch, A, B, C, ZA, ZB, bias, scale, fbias, nullptr, &act);
}

// og_int8_gemm's float product (or og_int8_gemm_float_scaled's, with act_scale given) that also records the range of
// what it stores, for og_dynamic_quantize_ranged (no counterpart in the reference).
int og_int8_gemm_float_ranged(og_ctx *ctx, const og_int8_gemm_params *p, uint32_t batch, og_buffer A, og_buffer B,
                              og_buffer C, og_buffer ZA, og_buffer ZB, og_buffer bias, og_buffer act_scale,
                              uint32_t act_offset, og_buffer scale, og_buffer fbias, og_buffer ranges, uint32_t *groups)
{
    const ActScale act{act_scale, act_offset};
    const RangeOut rout{ranges, groups};
    return run_gemm(ctx, p, batch, A, B, C, ZA, ZB, bias, scale, fbias, nullptr, act_scale.ptr ? &act : nullptr,
                    false, &rout);
}

int og_int8_gemm_requantized(og_ctx *ctx, const og_int8_gemm_params *p, uint32_t batch, og_buffer A, og_buffer B,
                             og_buffer Y, og_buffer ZA, og_buffer ZB, og_buffer bias, og_buffer multiplier,
                             int32_t zero_point_y, uint32_t y_signed)
{
    const RequantOut rq{zero_point_y, y_signed != 0};
    return run_gemm(ctx, p, batch, A, B, Y, ZA, ZB, bias, multiplier, og_buffer{nullptr, 0}, &rq);
}

int og_int8_epilogue(og_ctx *ctx, const og_int8_epilogue_params *p, og_buffer acc, og_buffer out, og_buffer bias,
                     og_buffer scale, og_buffer fbias)
{
    if (!p) return fail(ctx, OG_ERR_INVALID_ARG, "params", "null parameter block");
    if (p->Mode > 3) return fail(ctx, OG_ERR_INVALID_ARG, "Mode", "unknown mode %u", p->Mode);
    if (p->Count > 0x7FFFFFFFu) return fail(ctx, OG_ERR_INVALID_ARG, "Count", "too many elements");
    if (p->Count > 0 && p->N == 0) return fail(ctx, OG_ERR_INVALID_ARG, "N", "must be at least 1");
    const uint64_t cnt = p->Count, n = p->N;
    const bool byte_out = p->Mode == 2;
    if (p->Mode != 3) {
        if (cnt && (!acc.ptr || ((uintptr_t)acc.ptr & 3))) return fail(ctx, OG_ERR_INVALID_ARG, "scratch", "the int32 sums are missing or misaligned");
        if (cnt && !fits((uint64_t)p->OffAcc * 4, cnt * 4, acc)) return fail(ctx, OG_ERR_INVALID_ARG, "scratch", "elements %u..%llu reach past the buffer", p->OffAcc, (unsigned long long)(p->OffAcc + cnt));
    }
    if (cnt && (!out.ptr || (!byte_out && ((uintptr_t)out.ptr & 3)))) return fail(ctx, OG_ERR_INVALID_ARG, "y", "the output is missing or misaligned");
    if (cnt && !fits((uint64_t)p->OffOut * (byte_out ? 1 : 4), cnt * (byte_out ? 1 : 4), out)) return fail(ctx, OG_ERR_INVALID_ARG, "y", "elements %u..%llu reach past the buffer", p->OffOut, (unsigned long long)(p->OffOut + cnt));
    if ((p->Flags & 1u) && p->Mode != 3 && cnt && !fits((uint64_t)p->OffBias * 4, n * 4, bias)) return fail(ctx, OG_ERR_INVALID_ARG, "intBias", "the bias does not cover N values");
    if ((p->Mode == 1 || p->Mode == 2) && cnt && (!scale.ptr || !fits((uint64_t)p->OffScale * 4, ((p->Flags & 2u) ? n : 1) * 4, scale))) return fail(ctx, OG_ERR_INVALID_ARG, "multiplier", "the scale does not cover its values");
    if (p->Mode == 3 && cnt && (!fbias.ptr || !fits((uint64_t)p->OffFBias * 4, n * 4, fbias))) return fail(ctx, OG_ERR_INVALID_ARG, "floatBias", "the float bias does not cover N values");
    if (p->Mode == 2) {
        const bool u8 = p->Flags & 8u;
        if (p->ZeroPoint < (u8 ? 0 : -128) || p->ZeroPoint > (u8 ? 255 : 127)) return fail(ctx, OG_ERR_INVALID_ARG, "zeroPointY", "%d is outside the output type's range", p->ZeroPoint);
    }
    if (!ctx) return fail(ctx, OG_ERR_NO_DEVICE, "ctx", "no context: the arguments are valid but there is no device to run on");
    og::EpilogueArgs e{};
    e.acc = acc.ptr ? static_cast<const int32_t *>(acc.ptr) + p->OffAcc : nullptr;
    e.out = static_cast<uint8_t *>(out.ptr) + (uint64_t)p->OffOut * (byte_out ? 1 : 4);
    e.bias = (p->Flags & 1u) ? static_cast<const int32_t *>(bias.ptr) + p->OffBias : nullptr;
    e.scale = scale.ptr ? static_cast<const float *>(scale.ptr) + p->OffScale : nullptr;
    e.fbias = fbias.ptr ? static_cast<const float *>(fbias.ptr) + p->OffFBias : nullptr;
    e.count = p->Count;
    e.n = p->N;
    e.mode = p->Mode;
    e.flags = p->Flags;
    e.zero_point = p->ZeroPoint;
    e.out_byte_offset = byte_out ? p->OffOut : 0;
    (void)hipSetDevice(ctx->device);
    int st = launch(ctx, "og_int8_epilogue", [&](const char **k) { return og::launch_int8_epilogue(e, ctx->stream, k); });
    return st == OG_OK ? ok(ctx) : st;
}

// ------------------------------------------------------------------ ConvInteger

namespace {

// The geometry of a convolution after ConvKernels.CheckConv (ConvKernels.cs:895-956) and ConvIntegerKernels.Geometry
// (ConvIntegerKernels.cs:296-318); `arg` names what failed.
struct ConvGeometry {
    // kp: K padded to a multiple of 64 when 64 <= K and K % 64 != 0 (else K); cols_image: one image's column matrices;
    // wp_bytes: the padded weight copy ahead of them (0 without padding, with room to align its start to 16 bytes);
    // per_image = wp_bytes + cols_image, the scratch that one image needs.
    int64_t oh, ow, cin_g, cout_g, k, kp, ldb, cols_image, wp_bytes, per_image, x_image, y_image;
    const char *arg;
    const char *msg;
};

int64_t conv_extent(int64_t in, int64_t kernel, int64_t stride, int64_t dilation, int64_t pb, int64_t pe)
{
    const int64_t span = in + pb + pe - (dilation * (kernel - 1) + 1);
    return span < 0 ? 0 : span / stride + 1;
}

bool conv_geometry(const og_conv_params *p, ConvGeometry &g)
{
    const int64_t imax = 0x7FFFFFFF;
    g.arg = nullptr;
    auto bad = [&](const char *arg, const char *msg) { g.arg = arg; g.msg = msg; return false; };
    if (p->Batch < 1 || p->Batch > imax) return bad("Batch", "batch must be at least 1");
    if (p->InChannels < 1 || p->InChannels > imax) return bad("InChannels", "channel counts must be at least 1");
    if (p->OutChannels < 1 || p->OutChannels > imax) return bad("OutChannels", "channel counts must be at least 1");
    if (p->Groups < 1 || p->Groups > imax || p->InChannels % p->Groups || p->OutChannels % p->Groups)
        return bad("Groups", "the groups do not divide the input and output channels");
    const uint32_t in[2] = {p->Height, p->Width}, ker[2] = {p->KernelHeight, p->KernelWidth};
    const uint32_t str[2] = {p->StrideHeight, p->StrideWidth}, dil[2] = {p->DilationHeight, p->DilationWidth};
    const uint32_t pb[2] = {p->PadTop, p->PadLeft}, pe[2] = {p->PadBottom, p->PadRight};
    int64_t out[2];
    for (int a = 0; a < 2; a++) {
        const char *axis = a ? "width" : "height";
        if (in[a] < 1 || in[a] > imax) return bad(axis, "the input extent must be at least 1");
        if (ker[a] < 1 || ker[a] > imax) return bad(axis, "the kernel extent must be at least 1");
        if (str[a] < 1 || str[a] > imax) return bad(axis, "the stride must be at least 1");
        if (dil[a] < 1 || dil[a] > imax) return bad(axis, "the dilation must be at least 1");
        if (pb[a] > imax || pe[a] > imax) return bad(axis, "the padding must not be negative");
        if ((int64_t)ker[a] * dil[a] > imax || (int64_t)pb[a] + pe[a] + in[a] > imax)
            return bad(axis, "the window or padding is larger than the supported sizes");
        out[a] = conv_extent(in[a], ker[a], str[a], dil[a], pb[a], pe[a]);
        if (out[a] < 1) return bad(axis, "the kernel does not fit the padded input");
    }
    g.oh = out[0];
    g.ow = out[1];
    g.cin_g = p->InChannels / p->Groups;
    g.cout_g = p->OutChannels / p->Groups;
    g.k = g.cin_g * p->KernelHeight * p->KernelWidth;
    g.ldb = (g.oh * g.ow + 15) / 16 * 16;
    g.x_image = (int64_t)p->InChannels * p->Height * p->Width;
    g.y_image = (int64_t)p->OutChannels * g.oh * g.ow;
    if (g.k > imax || g.ldb > imax || g.x_image * p->Batch > imax) return bad("shape", "the convolution is larger than the supported sizes");
    const bool pad = g.k >= 64 && g.k % 64 != 0;
    g.kp = pad ? (g.k + 63) / 64 * 64 : g.k;
    g.cols_image = (int64_t)p->Groups * g.kp * g.ldb;
    g.wp_bytes = pad ? 16 + ((int64_t)p->OutChannels * g.kp + 255) / 256 * 256 : 0;
    g.per_image = g.wp_bytes + g.cols_image;
    if (g.kp > imax || g.per_image > imax)
        return bad("InChannels", "the column matrix of one image is larger than the supported sizes");
    return true;
}

}  // namespace

uint64_t og_conv_integer_scratch_bytes(const og_conv_params *p)
{
    ConvGeometry g;
    return p && conv_geometry(p, g) ? (uint64_t)g.per_image : 0;
}

int og_conv_integer(og_ctx *ctx, const og_conv_params *p, og_buffer x, og_buffer w, og_buffer y, og_buffer xz,
                    og_buffer wz, og_buffer scratch, uint64_t scratch_offset)
{
    if (!p) return fail(ctx, OG_ERR_INVALID_ARG, "params", "null parameter block");
    ConvGeometry geo;
    if (!conv_geometry(p, geo)) return fail(ctx, OG_ERR_INVALID_ARG, geo.arg, "%s", geo.msg);
    const uint32_t known = OG_CONV_X_INT8 | OG_CONV_W_INT8 | OG_CONV_XZ | OG_CONV_WZ | OG_CONV_WZ_PER_CHANNEL | OG_CONV_NO_DEPTHWISE;
    if (p->Flags & ~known) return fail(ctx, OG_ERR_INVALID_ARG, "Flags", "unknown flag bits 0x%x", p->Flags & ~known);
    const uint32_t gemm_known =
        OG_GEMM_PORTABLE | OG_GEMM_NO_SKINNY | OG_GEMM_NO_DIRECT | OG_GEMM_LARGE_TILE | OG_GEMM_NO_STREAM | OG_GEMM_TWO_PASS;
    if (p->GemmFlags & ~gemm_known) return fail(ctx, OG_ERR_INVALID_ARG, "GemmFlags", "flag bits 0x%x are not product options", p->GemmFlags & ~gemm_known);
    if ((p->Flags & OG_CONV_WZ_PER_CHANNEL) && !(p->Flags & OG_CONV_WZ)) return fail(ctx, OG_ERR_INVALID_ARG, "Flags", "a per-channel zero point without a zero point");
    const int64_t B = p->Batch;
    if (!x.ptr || !fits(p->OffsetX, (uint64_t)(geo.x_image * B), x)) return fail(ctx, OG_ERR_INVALID_ARG, "x", "elements %u..%lld reach past the buffer", p->OffsetX, (long long)(p->OffsetX + geo.x_image * B));
    if (!w.ptr || !fits(p->OffsetW, (uint64_t)(p->OutChannels * geo.k), w)) return fail(ctx, OG_ERR_INVALID_ARG, "w", "elements %u..%lld reach past the buffer", p->OffsetW, (long long)(p->OffsetW + p->OutChannels * geo.k));
    if ((int64_t)p->OffsetY + geo.y_image * B > 0x7FFFFFFF) return fail(ctx, OG_ERR_INVALID_ARG, "y", "the result is larger than the supported sizes");
    if (!y.ptr || ((uintptr_t)y.ptr & 3) || !fits((uint64_t)p->OffsetY * 4, (uint64_t)(geo.y_image * B) * 4, y)) return fail(ctx, OG_ERR_INVALID_ARG, "y", "elements %u..%lld reach past the buffer (or it is misaligned)", p->OffsetY, (long long)(p->OffsetY + geo.y_image * B));
    if ((p->Flags & OG_CONV_XZ) && (!xz.ptr || !fits(p->OffXZero, 1, xz))) return fail(ctx, OG_ERR_INVALID_ARG, "xZeroPoint", "element %u reaches past the buffer", p->OffXZero);
    const uint64_t nwz = (p->Flags & OG_CONV_WZ_PER_CHANNEL) ? p->OutChannels : 1;
    if ((p->Flags & OG_CONV_WZ) && (!wz.ptr || !fits(p->OffWZero, nwz, wz))) return fail(ctx, OG_ERR_INVALID_ARG, "wZeroPoint", "elements %u..%llu reach past the buffer", p->OffWZero, (unsigned long long)(p->OffWZero + nwz));
    const bool depthwise = geo.cin_g == 1 && !(p->Flags & OG_CONV_NO_DEPTHWISE);
    // A 1 x 1 window with unit strides and no padding: image n's channels of group g already are the product's B
    // operand, [cin_g x H*W] in rows of H*W bytes, so there is nothing to pack, as long as those rows suit the
    // LDS-DMA kernel (whole 16-byte chunks from a 16-byte aligned start); otherwise the packed copy, whose rows are
    // padded to 16 bytes, is the faster operand.
    const int64_t plane = (int64_t)p->Height * p->Width;
    const bool pointwise = !depthwise && p->KernelHeight == 1 && p->KernelWidth == 1 && p->StrideHeight == 1 &&
                           p->StrideWidth == 1 && p->PadTop == 0 && p->PadLeft == 0 && p->PadBottom == 0 &&
                           p->PadRight == 0 && plane % 16 == 0 &&
                           ((uintptr_t)static_cast<const uint8_t *>(x.ptr) + p->OffsetX) % 16 == 0;
    int64_t per_chunk = B;
    if (!depthwise && !pointwise) {
        if (scratch_offset & 3) return fail(ctx, OG_ERR_INVALID_ARG, "scratchOffset", "offset %llu must be a multiple of 4", (unsigned long long)scratch_offset);
        if (!scratch.ptr || !fits(scratch_offset, (uint64_t)geo.per_image, scratch)) return fail(ctx, OG_ERR_INVALID_ARG, "scratch", "one image's columns (%lld bytes from %llu) reach past the buffer", (long long)geo.per_image, (unsigned long long)scratch_offset);
        per_chunk = std::min<int64_t>(B, (int64_t)(scratch.bytes - scratch_offset - (uint64_t)geo.wp_bytes) / geo.cols_image);
        per_chunk = std::min<int64_t>(per_chunk, 0x7FFFFFFF / geo.cols_image);   // one chunk's columns stay under 2 GiB
    }
    if (!ctx) return fail(ctx, OG_ERR_NO_DEVICE, "ctx", "no context: the arguments are valid but there is no device to run on");
    (void)hipSetDevice(ctx->device);

    const uint8_t *xb = static_cast<const uint8_t *>(x.ptr) + p->OffsetX;
    const uint8_t *wb = static_cast<const uint8_t *>(w.ptr) + p->OffsetW;
    int32_t *yb = static_cast<int32_t *>(y.ptr) + p->OffsetY;
    const uint8_t *xzp = (p->Flags & OG_CONV_XZ) ? static_cast<const uint8_t *>(xz.ptr) + p->OffXZero : nullptr;
    const uint8_t *wzp = (p->Flags & OG_CONV_WZ) ? static_cast<const uint8_t *>(wz.ptr) + p->OffWZero : nullptr;
    int st = OG_OK;
    if (depthwise) {
        og::ConvDepthwiseArgs a{};
        a.x = xb;
        a.wt = wb;
        a.xz = xzp;
        a.wz = wzp;
        a.y = yb;
        a.batch = (int32_t)B;
        a.cin = (int32_t)p->InChannels;
        a.cout = (int32_t)p->OutChannels;
        a.h = (int32_t)p->Height;
        a.w = (int32_t)p->Width;
        a.oh = (int32_t)geo.oh;
        a.ow = (int32_t)geo.ow;
        a.kh = (int32_t)p->KernelHeight;
        a.kw = (int32_t)p->KernelWidth;
        a.sh = (int32_t)p->StrideHeight;
        a.sw = (int32_t)p->StrideWidth;
        a.dh = (int32_t)p->DilationHeight;
        a.dw = (int32_t)p->DilationWidth;
        a.ph = (int32_t)p->PadTop;
        a.pw = (int32_t)p->PadLeft;
        a.x_signed = p->Flags & OG_CONV_X_INT8;
        a.w_signed = p->Flags & OG_CONV_W_INT8;
        a.wz_per_channel = p->Flags & OG_CONV_WZ_PER_CHANNEL;
        st = launch(ctx, "og_conv_integer", [&](const char **k) { return og::launch_conv_depthwise(a, ctx->stream, k); });
        return st == OG_OK ? ok(ctx) : st;
    }
    const int64_t ncols = geo.oh * geo.ow;
    // The products: A = group g's weights [cout_g x k] (its zero point per row = per output channel), B = the group's
    // column matrix [k x ncols] (x's zero point), one batch entry per image.
    // a / kk: the weights and their row length (the padded copy and kp after a padded pack).
    auto product = [&](const uint8_t *a, int64_t kk, const uint8_t *b, int64_t ldb, int64_t stride_b, int64_t b_bytes,
                       int64_t first, int32_t images, int64_t g) {
        og::GemmArgs ga{};
        ga.A = a + g * geo.cout_g * kk;
        ga.B = b;
        ga.C = yb + first * geo.y_image + g * geo.cout_g * ncols;
        ga.ZA = wzp ? wzp + ((p->Flags & OG_CONV_WZ_PER_CHANNEL) ? g * geo.cout_g : 0) : nullptr;
        ga.ZB = xzp;
        ga.strideA = 0;
        ga.strideB = stride_b;
        ga.strideC = geo.y_image;
        ga.b_bytes = b_bytes;
        ga.M = (int32_t)geo.cout_g;
        ga.N = (int32_t)ncols;
        ga.K = (int32_t)kk;
        ga.batch = images;
        ga.lda = (int32_t)kk;
        ga.ldb = (int32_t)ldb;
        ga.flags = p->GemmFlags | ((p->Flags & OG_CONV_W_INT8) ? OG_GEMM_A_INT8 : 0u) |
                   ((p->Flags & OG_CONV_X_INT8) ? OG_GEMM_B_INT8 : 0u) | (wzp ? OG_GEMM_ZA : 0u) |
                   ((p->Flags & OG_CONV_WZ_PER_CHANNEL) ? OG_GEMM_ZA_PER_ROW : 0u) | (xzp ? OG_GEMM_ZB : 0u);
        ga.epi = 0;
        return launch_product(ctx, ga);
    };
    if (pointwise) {
        for (int64_t g = 0; g < p->Groups && st == OG_OK; g++)
            st = product(wb, geo.k, xb + g * geo.cin_g * plane, plane, geo.x_image,
                         (int64_t)(x.bytes - p->OffsetX) - g * geo.cin_g * plane, 0, (int32_t)B, g);
        return st == OG_OK ? ok(ctx) : st;
    }
    // Scratch: [the padded weights, from the first 16-byte boundary] [the column matrices of a chunk of images].
    uint8_t *const base = static_cast<uint8_t *>(scratch.ptr) + scratch_offset;
    uint8_t *const wp = geo.wp_bytes ? reinterpret_cast<uint8_t *>(((uintptr_t)base + 15) & ~(uintptr_t)15) : nullptr;
    uint8_t *const cols = geo.wp_bytes ? wp + (geo.wp_bytes - 16) : base;
    const int64_t cols_room = (int64_t)scratch.bytes - (int64_t)(cols - static_cast<uint8_t *>(scratch.ptr));
    for (int64_t first = 0; first < B && st == OG_OK; first += per_chunk) {
        const int32_t images = (int32_t)std::min<int64_t>(per_chunk, B - first);
        og::ConvPackArgs pa{};
        pa.x = xb + first * geo.x_image;
        pa.xz = xzp;
        pa.cols = cols;
        pa.images = images;
        pa.groups = (int32_t)p->Groups;
        pa.k = (int32_t)geo.k;
        pa.cin = (int32_t)p->InChannels;
        pa.cin_g = (int32_t)geo.cin_g;
        pa.h = (int32_t)p->Height;
        pa.w = (int32_t)p->Width;
        pa.oh = (int32_t)geo.oh;
        pa.ow = (int32_t)geo.ow;
        pa.kh = (int32_t)p->KernelHeight;
        pa.kw = (int32_t)p->KernelWidth;
        pa.sh = (int32_t)p->StrideHeight;
        pa.sw = (int32_t)p->StrideWidth;
        pa.dh = (int32_t)p->DilationHeight;
        pa.dw = (int32_t)p->DilationWidth;
        pa.ph = (int32_t)p->PadTop;
        pa.pw = (int32_t)p->PadLeft;
        pa.ldb = geo.ldb;
        pa.kp = (int32_t)geo.kp;
        pa.wrows = geo.wp_bytes && first == 0 ? (int32_t)p->OutChannels : 0;   // the weights once, with the first chunk
        pa.wt = wb;
        pa.wp = wp;
        st = launch(ctx, "og_conv_integer", [&](const char **k) { return og::launch_conv_pack(pa, ctx->stream, k); });
        for (int64_t g = 0; g < p->Groups && st == OG_OK; g++)
            st = product(geo.wp_bytes ? wp : wb, geo.kp, cols + g * geo.kp * geo.ldb, geo.ldb, p->Groups * geo.kp * geo.ldb,
                         cols_room - g * geo.kp * geo.ldb, first, images, g);
    }
    return st == OG_OK ? ok(ctx) : st;
}

// ------------------------------------------------------------------ Gather

int og_gather(og_ctx *ctx, uint32_t elem_bytes, const og_gather_params *p, og_buffer data, og_buffer indices,
              og_buffer out, og_buffer status)
{
    if (!p) return fail(ctx, OG_ERR_INVALID_ARG, "params", "null parameter block");
    if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8)
        return fail(ctx, OG_ERR_INVALID_ARG, "T", "element size %u is not 1, 2, 4 or 8 bytes", elem_bytes);
    if (p->Flags & ~1u) return fail(ctx, OG_ERR_INVALID_ARG, "Flags", "unknown flag bits 0x%x", p->Flags & ~1u);
    if (p->Count > 0x7FFFFFFFu) return fail(ctx, OG_ERR_INVALID_ARG, "indexCount", "the output holds more elements than the kernels address");
    const uint64_t per_outer = (uint64_t)p->IdxCount * p->Inner;
    if (per_outer == 0 ? p->Count != 0 : p->Count % per_outer != 0)
        return fail(ctx, OG_ERR_INVALID_ARG, "Count", "%u is not a multiple of IdxCount * Inner = %llu", p->Count, (unsigned long long)per_outer);
    if (p->AxisLen > 0x7FFFFFFFu) return fail(ctx, OG_ERR_INVALID_ARG, "AxisLen", "the axis is longer than an index reaches");
    const uint64_t outer = per_outer ? p->Count / per_outer : 0;
    const bool wide = p->Flags & 1u;
    const uint64_t eb = elem_bytes;
    if (p->Count > 0) {
        const uint64_t data_elems = outer * p->AxisLen * p->Inner;
        if (data_elems > 0 && (!data.ptr || !fits((uint64_t)p->OffData * eb, data_elems * eb, data)))
            return fail(ctx, OG_ERR_INVALID_ARG, "data", "elements %u..%llu reach past the buffer", p->OffData, (unsigned long long)(p->OffData + data_elems));
        const uint64_t ib = wide ? 8 : 4;
        if (!indices.ptr || ((uintptr_t)indices.ptr & 3) || !fits((uint64_t)p->OffIdx * ib, (uint64_t)p->IdxCount * ib, indices))
            return fail(ctx, OG_ERR_INVALID_ARG, "indices", "elements %u..%llu reach past the buffer", p->OffIdx, (unsigned long long)p->OffIdx + p->IdxCount);
        if (!out.ptr || !fits((uint64_t)p->OffOut * eb, (uint64_t)p->Count * eb, out))
            return fail(ctx, OG_ERR_INVALID_ARG, "output", "elements %u..%llu reach past the buffer", p->OffOut, (unsigned long long)p->OffOut + p->Count);
        if (status.ptr && (((uintptr_t)status.ptr & 3) || status.bytes < 4))
            return fail(ctx, OG_ERR_INVALID_ARG, "status", "the status word is misaligned or too small");
        // With an empty axis every index is invalid and the data is never read (it may be absent).
    }
    if (!ctx) return fail(ctx, OG_ERR_NO_DEVICE, "ctx", "no context: the arguments are valid but there is no device to run on");
    if (p->Count == 0) return ok(ctx);
    og::GatherArgs a{};
    a.data = static_cast<const uint8_t *>(data.ptr) + (uint64_t)p->OffData * eb;
    a.idx = static_cast<const uint8_t *>(indices.ptr) + (uint64_t)p->OffIdx * (wide ? 8 : 4);
    a.out = static_cast<uint8_t *>(out.ptr) + (uint64_t)p->OffOut * eb;
    a.status = static_cast<uint32_t *>(status.ptr);
    a.rows = (int64_t)(outer * p->IdxCount);
    a.count = p->IdxCount;
    a.axis_len = p->AxisLen;
    a.row_bytes = (int64_t)p->Inner * (int64_t)eb;
    a.wide = wide;
    (void)hipSetDevice(ctx->device);
    int st = launch(ctx, "og_gather", [&](const char **k) { return og::launch_gather(a, ctx->stream, k); });
    return st == OG_OK ? ok(ctx) : st;
}

// ------------------------------------------------------------------ DynamicQuantizeLinear

// DynamicQuantizeLinear's argument checks (DynamicQuantizeKernels.cs:59-90) and its resolved arguments.
static int dq_args(og_ctx *ctx, const og_dq_params *p, og_buffer X, og_buffer Y, og_buffer scale, og_buffer zero,
                   og::DqArgs *d)
{
    if (!p) return fail(ctx, OG_ERR_INVALID_ARG, "params", "null parameter block");
    if (p->Count < 1 || p->Count > 0x7FFFFFFFu) return fail(ctx, OG_ERR_INVALID_ARG, "count", "count %d must be at least 1", (int32_t)p->Count);
    if (!X.ptr || ((uintptr_t)X.ptr & 3) || !fits((uint64_t)p->OffX * 4, (uint64_t)p->Count * 4, X)) return fail(ctx, OG_ERR_INVALID_ARG, "x", "elements %u..%llu reach past the buffer", p->OffX, (unsigned long long)p->OffX + p->Count);
    if (!Y.ptr || !fits(p->OffY, p->Count, Y)) return fail(ctx, OG_ERR_INVALID_ARG, "y", "elements %u..%llu reach past the buffer", p->OffY, (unsigned long long)p->OffY + p->Count);
    if (!scale.ptr || ((uintptr_t)scale.ptr & 3) || !fits((uint64_t)p->OffScale * 4, 4, scale)) return fail(ctx, OG_ERR_INVALID_ARG, "scale", "element %u reaches past the buffer", p->OffScale);
    if (!zero.ptr || !fits(p->OffZero, 1, zero)) return fail(ctx, OG_ERR_INVALID_ARG, "zeroPoint", "element %u reaches past the buffer", p->OffZero);
    *d = og::DqArgs{};
    d->x = static_cast<const float *>(X.ptr) + p->OffX;
    d->y = static_cast<uint8_t *>(Y.ptr) + p->OffY;
    d->scale = static_cast<float *>(scale.ptr) + p->OffScale;
    d->zero = static_cast<uint8_t *>(zero.ptr) + p->OffZero;
    d->count = p->Count;
    return OG_OK;
}

int og_dynamic_quantize(og_ctx *ctx, const og_dq_params *p, og_buffer X, og_buffer Y, og_buffer scale, og_buffer zero)
{
    og::DqArgs d{};
    int st0 = dq_args(ctx, p, X, Y, scale, zero, &d);
    if (st0 != OG_OK) return st0;
    if (!ctx) return fail(ctx, OG_ERR_NO_DEVICE, "ctx", "no context: the arguments are valid but there is no device to run on");
    (void)hipSetDevice(ctx->device);
    int st = launch(ctx, "og_dynamic_quantize", [&](const char **k) { return og::launch_dynamic_quantize(d, ctx->ws, ctx->stream, k, 0); });
    if (st == OG_OK) st = launch(ctx, "og_dynamic_quantize", [&](const char **k) { return og::launch_dynamic_quantize(d, ctx->ws, ctx->stream, k, 1); });
    return st == OG_OK ? ok(ctx) : st;
}

// DynamicQuantizeLinear's quantize pass alone, over the ranges a ranged product recorded for x (no counterpart in the
// reference).
int og_dynamic_quantize_ranged(og_ctx *ctx, const og_dq_params *p, og_buffer X, og_buffer Y, og_buffer scale,
                               og_buffer zero, og_buffer ranges, uint32_t groups)
{
    og::DqArgs d{};
    int st0 = dq_args(ctx, p, X, Y, scale, zero, &d);
    if (st0 != OG_OK) return st0;
    if (!ranges.ptr || ((uintptr_t)ranges.ptr & 7) || ranges.bytes < 8ull * og::kRangesMax) return fail(ctx, OG_ERR_INVALID_ARG, "ranges", "the ranges need %d (min, max) pairs of float32, 8-byte aligned", og::kRangesMax);
    if (groups < 1 || groups > (uint32_t)og::kRangesMax) return fail(ctx, OG_ERR_INVALID_ARG, "groups", "%u pairs: between 1 and %d", groups, og::kRangesMax);
    if (!ctx) return fail(ctx, OG_ERR_NO_DEVICE, "ctx", "no context: the arguments are valid but there is no device to run on");
    (void)hipSetDevice(ctx->device);
    int st = launch(ctx, "og_dynamic_quantize_ranged", [&](const char **k) {
        return og::launch_dynamic_quantize_ranged(d, static_cast<const float *>(ranges.ptr), groups, ctx->stream, k);
    });
    return st == OG_OK ? ok(ctx) : st;
}

// ------------------------------------------------------------------ DequantizeLinear / QuantizeLinear

static int check_axis(og_ctx *ctx, const og_dequant_params *p)
{
    if (p->Count > 0x7FFFFFFFu) return fail(ctx, OG_ERR_INVALID_ARG, "shape", "the tensor holds more than 2147483647 elements");
    if (p->Flags & ~3u) return fail(ctx, OG_ERR_INVALID_ARG, "Flags", "unknown flag bits 0x%x", p->Flags & ~3u);
    if ((p->Flags & 1u) && (p->AxisLen == 0 || p->Inner == 0) && p->Count) return fail(ctx, OG_ERR_INVALID_ARG, "axis", "per-axis parameters need AxisLen and Inner of at least 1");
    return OG_OK;
}

// Checks one DequantizeLinear pass and forms its kernel arguments.
static int dequant_args(og_ctx *ctx, int kind, int f16_out, const og_dequant_params *p, og_buffer X, og_buffer scale,
                        og_buffer zero, og_buffer out, og::DequantArgs *d)
{
    if (!p) return fail(ctx, OG_ERR_INVALID_ARG, "params", "null parameter block");
    if (kind < OG_KIND_U8 || kind > OG_KIND_I32) return fail(ctx, OG_ERR_INVALID_ARG, "TIn", "unknown input kind %d", kind);
    int st = check_axis(ctx, p);
    if (st != OG_OK) return st;
    const uint64_t cnt = p->Count, params = (p->Flags & 1u) ? p->AxisLen : 1, esz = kind == OG_KIND_I32 ? 4 : 1;
    const uint64_t osz = f16_out ? 2 : 4;
    if (cnt) {
        if (!X.ptr || (esz == 4 && ((uintptr_t)X.ptr & 3)) || !fits(p->OffX * esz, cnt * esz, X)) return fail(ctx, OG_ERR_INVALID_ARG, "x", "elements %u..%llu reach past the buffer", p->OffX, (unsigned long long)(p->OffX + cnt));
        if (!scale.ptr || ((uintptr_t)scale.ptr & 3) || !fits((uint64_t)p->OffS * 4, params * 4, scale)) return fail(ctx, OG_ERR_INVALID_ARG, "scale", "elements %u..%llu reach past the buffer", p->OffS, (unsigned long long)(p->OffS + params));
        if ((p->Flags & 2u) && (!zero.ptr || (esz == 4 && ((uintptr_t)zero.ptr & 3)) || !fits(p->OffZ * esz, params * esz, zero))) return fail(ctx, OG_ERR_INVALID_ARG, "zeroPoint", "elements %u..%llu reach past the buffer", p->OffZ, (unsigned long long)(p->OffZ + params));
        if (!out.ptr || ((uintptr_t)out.ptr & (osz - 1)) || !fits(p->OffO * osz, cnt * osz, out)) return fail(ctx, OG_ERR_INVALID_ARG, "output", "elements %u..%llu reach past the buffer", p->OffO, (unsigned long long)(p->OffO + cnt));
    }
    *d = og::DequantArgs{};
    d->x = static_cast<const uint8_t *>(X.ptr) + p->OffX * esz;
    d->scale = static_cast<const float *>(scale.ptr) + p->OffS;
    d->zero = (p->Flags & 2u) ? static_cast<const uint8_t *>(zero.ptr) + p->OffZ * esz : nullptr;
    d->out = static_cast<uint8_t *>(out.ptr) + p->OffO * osz;
    d->count = p->Count;
    d->axis_len = p->AxisLen ? p->AxisLen : 1;
    d->inner = p->Inner ? p->Inner : 1;
    d->per_axis = p->Flags & 1u;
    d->has_zero = p->Flags & 2u;
    return OG_OK;
}

int og_dequantize(og_ctx *ctx, int kind, int f16_out, const og_dequant_params *p, og_buffer X, og_buffer scale,
                  og_buffer zero, og_buffer out)
{
    og::DequantArgs d;
    int st = dequant_args(ctx, kind, f16_out, p, X, scale, zero, out, &d);
    if (st != OG_OK) return st;
    if (!ctx) return fail(ctx, OG_ERR_NO_DEVICE, "ctx", "no context: the arguments are valid but there is no device to run on");
    (void)hipSetDevice(ctx->device);
    st = launch(ctx, "og_dequantize", [&](const char **k) { return og::launch_dequantize(d, kind, f16_out != 0, ctx->stream, k); });
    return st == OG_OK ? ok(ctx) : st;
}

int og_dequantize_batch(og_ctx *ctx, int kind, int f16_out, uint32_t n, const og_dequant_params *params,
                        const og_buffer *X, const og_buffer *scale, const og_buffer *zero, const og_buffer *out)
{
    if (n == 0) return ok(ctx);
    if (!params || !X || !scale || !zero || !out) return fail(ctx, OG_ERR_INVALID_ARG, "params", "null array");
    if (n > OG_DEQUANT_BATCH_MAX) return fail(ctx, OG_ERR_INVALID_ARG, "n", "%u passes; at most %u a call", n, (unsigned)OG_DEQUANT_BATCH_MAX);
    std::vector<og::DequantArgs> d(n);
    for (uint32_t i = 0; i < n; i++) {
        const og_dequant_params &a = params[0], &b = params[i];
        if (b.Count != a.Count || b.Flags != a.Flags || ((b.Flags & 1u) && (b.AxisLen != a.AxisLen || b.Inner != a.Inner)))
            return fail(ctx, OG_ERR_INVALID_ARG, "params", "pass %u's count, flags or axis differ from pass 0's", i);
        const int st = dequant_args(ctx, kind, f16_out, &b, X[i], scale[i], zero[i], out[i], &d[i]);
        if (st != OG_OK) return st;
    }
    // Passes run together, so no pass may write what another reads or writes.
    const uint64_t esz = kind == OG_KIND_I32 ? 4 : 1, osz = f16_out ? 2 : 4;
    const uint64_t pbytes = (params[0].Flags & 1u) ? (uint64_t)params[0].AxisLen * 4 : 4;
    const uint64_t zbytes = (params[0].Flags & 1u) ? (uint64_t)params[0].AxisLen * esz : esz;
    auto overlap = [](const void *a, uint64_t an, const void *b, uint64_t bn) {
        const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
        return an && bn && x < y + bn && y < x + an;
    };
    const uint64_t cnt = params[0].Count;
    for (uint32_t i = 0; i < n; i++)
        for (uint32_t j = 0; j < n; j++) {
            if (i == j) continue;
            const bool hit = overlap(d[i].out, cnt * osz, d[j].x, cnt * esz) || overlap(d[i].out, cnt * osz, d[j].scale, pbytes) ||
                             (d[j].has_zero && overlap(d[i].out, cnt * osz, d[j].zero, zbytes)) ||
                             overlap(d[i].out, cnt * osz, d[j].out, cnt * osz);
            if (hit) return fail(ctx, OG_ERR_INVALID_ARG, "output", "pass %u's output overlaps pass %u's operands", i, j);
        }
    if (!ctx) return fail(ctx, OG_ERR_NO_DEVICE, "ctx", "no context: the arguments are valid but there is no device to run on");
    (void)hipSetDevice(ctx->device);
    int st = launch(ctx, "og_dequantize_batch", [&](const char **k) {
        return og::launch_dequantize_batch(d.data(), (int)n, kind, f16_out != 0, ctx->stream, k);
    });
    return st == OG_OK ? ok(ctx) : st;
}

int og_quantize(og_ctx *ctx, int is_signed, int f16_in, const og_dequant_params *p, og_buffer X, og_buffer scale,
                og_buffer zero, og_buffer out)
{
    if (!p) return fail(ctx, OG_ERR_INVALID_ARG, "params", "null parameter block");
    int st = check_axis(ctx, p);
    if (st != OG_OK) return st;
    const uint64_t cnt = p->Count, params = (p->Flags & 1u) ? p->AxisLen : 1, isz = f16_in ? 2 : 4;
    if (cnt) {
        if (!X.ptr || ((uintptr_t)X.ptr & (isz - 1)) || !fits(p->OffX * isz, cnt * isz, X)) return fail(ctx, OG_ERR_INVALID_ARG, "x", "elements %u..%llu reach past the buffer", p->OffX, (unsigned long long)(p->OffX + cnt));
        if (!scale.ptr || ((uintptr_t)scale.ptr & 3) || !fits((uint64_t)p->OffS * 4, params * 4, scale)) return fail(ctx, OG_ERR_INVALID_ARG, "scale", "elements %u..%llu reach past the buffer", p->OffS, (unsigned long long)(p->OffS + params));
        if ((p->Flags & 2u) && (!zero.ptr || !fits(p->OffZ, params, zero))) return fail(ctx, OG_ERR_INVALID_ARG, "zeroPoint", "elements %u..%llu reach past the buffer", p->OffZ, (unsigned long long)(p->OffZ + params));
        if (!out.ptr || !fits(p->OffO, cnt, out)) return fail(ctx, OG_ERR_INVALID_ARG, "output", "elements %u..%llu reach past the buffer", p->OffO, (unsigned long long)(p->OffO + cnt));
    }
    if (!ctx) return fail(ctx, OG_ERR_NO_DEVICE, "ctx", "no context: the arguments are valid but there is no device to run on");
    og::DequantArgs d{};
    d.x = static_cast<const uint8_t *>(X.ptr) + p->OffX * isz;
    d.scale = static_cast<const float *>(scale.ptr) + p->OffS;
    d.zero = (p->Flags & 2u) ? static_cast<const uint8_t *>(zero.ptr) + p->OffZ : nullptr;
    d.out = static_cast<uint8_t *>(out.ptr) + p->OffO;
    d.count = p->Count;
    d.axis_len = p->AxisLen ? p->AxisLen : 1;
    d.inner = p->Inner ? p->Inner : 1;
    d.per_axis = p->Flags & 1u;
    d.has_zero = p->Flags & 2u;
    (void)hipSetDevice(ctx->device);
    st = launch(ctx, "og_quantize", [&](const char **k) { return og::launch_quantize(d, is_signed != 0, f16_in != 0, ctx->stream, k); });
    return st == OG_OK ? ok(ctx) : st;
}

// ------------------------------------------------------------------ utilities

int og_util_synth(og_ctx *ctx, int kind, uint64_t seed, uint32_t tensor, og_buffer out, uint64_t offset, uint64_t count,
                  double lo, double hi)
{
    if (kind < 0 || kind > 2) return fail(ctx, OG_ERR_INVALID_ARG, "kind", "unknown kind %d", kind);
    const uint64_t esz = kind == 0 ? 1 : 4;
    if (count && (!out.ptr || ((uintptr_t)out.ptr & (esz - 1)) || !fits(offset * esz, count * esz, out))) return fail(ctx, OG_ERR_INVALID_ARG, "out", "elements reach past the buffer");
    if (kind != 2 && (lo > hi || lo < -2147483648.0 || hi > 2147483647.0)) return fail(ctx, OG_ERR_INVALID_ARG, "lo", "bad integer range");
    if (!ctx) return fail(ctx, OG_ERR_NO_DEVICE, "ctx", "no context");
    (void)hipSetDevice(ctx->device);
    int st = launch(ctx, "og_util_synth", [&](const char **k) { *k = "synth"; return og::launch_synth(kind, seed, tensor, static_cast<uint8_t *>(out.ptr) + offset * esz, count, lo, hi, ctx->stream); });
    return st == OG_OK ? ok(ctx) : st;
}

int og_util_col_absmax_scale(og_ctx *ctx, og_buffer W, uint32_t rows, uint32_t cols, float divisor, og_buffer scale)
{
    if ((uint64_t)rows * cols && (!W.ptr || !fits(0, (uint64_t)rows * cols * 4, W))) return fail(ctx, OG_ERR_INVALID_ARG, "W", "the tensor reaches past the buffer");
    if (cols && (!scale.ptr || !fits(0, (uint64_t)cols * 4, scale))) return fail(ctx, OG_ERR_INVALID_ARG, "scale", "the scales reach past the buffer");
    if (!ctx) return fail(ctx, OG_ERR_NO_DEVICE, "ctx", "no context");
    (void)hipSetDevice(ctx->device);
    int st = launch(ctx, "og_util_col_absmax_scale", [&](const char **k) { *k = "col-absmax-scale"; return og::launch_col_absmax_scale(static_cast<const float *>(W.ptr), rows, cols, divisor, static_cast<float *>(scale.ptr), ctx->stream); });
    return st == OG_OK ? ok(ctx) : st;
}

int og_util_scale_product(og_ctx *ctx, og_buffer a, og_buffer b, uint32_t n, og_buffer out)
{
    if (n && (!a.ptr || !fits(0, 4, a) || !b.ptr || !fits(0, (uint64_t)n * 4, b) || !out.ptr || !fits(0, (uint64_t)n * 4, out))) return fail(ctx, OG_ERR_INVALID_ARG, "out", "operands do not cover n values");
    if (!ctx) return fail(ctx, OG_ERR_NO_DEVICE, "ctx", "no context");
    (void)hipSetDevice(ctx->device);
    int st = launch(ctx, "og_util_scale_product", [&](const char **k) { *k = "scale-product"; return og::launch_scale_product(static_cast<const float *>(a.ptr), static_cast<const float *>(b.ptr), n, static_cast<float *>(out.ptr), ctx->stream); });
    return st == OG_OK ? ok(ctx) : st;
}

int og_util_stream_tiles(og_ctx *ctx, og_buffer B, uint32_t K, uint32_t N, og_buffer sink)
{
    if (K < 1 || N < 16 || N % 16 || (uint64_t)K * N > 0x7FFFFFFFull) return fail(ctx, OG_ERR_INVALID_ARG, "K", "K >= 1, N >= 16 a multiple of 16, K * N < 2^31");
    if (!B.ptr || ((uintptr_t)B.ptr & 15) || !fits(0, (uint64_t)K * N, B)) return fail(ctx, OG_ERR_INVALID_ARG, "B", "B reaches past the buffer or is not 16-byte aligned");
    if (!sink.ptr || ((uintptr_t)sink.ptr & 3) || !fits(0, 4, sink)) return fail(ctx, OG_ERR_INVALID_ARG, "sink", "the sink needs 4 aligned bytes");
    if (!ctx) return fail(ctx, OG_ERR_NO_DEVICE, "ctx", "no context");
    (void)hipSetDevice(ctx->device);
    int st = launch(ctx, "og_util_stream_tiles", [&](const char **k) { *k = "stream-tiles"; return og::launch_stream_tiles(static_cast<const uint8_t *>(B.ptr), (int32_t)K, (int32_t)N, static_cast<uint32_t *>(sink.ptr), ctx->stream); });
    return st == OG_OK ? ok(ctx) : st;
}

// ------------------------------------------------------------------ test hooks

int og_test_set_spin_limit(og_ctx *ctx, uint32_t polls)
{
    if (!ctx) return fail(ctx, OG_ERR_INVALID_ARG, "ctx", "null context");
    ctx->spin_limit = polls;
    return ok(ctx);
}

int og_test_nonzero_words(og_ctx *ctx, uint64_t *context_words, uint64_t *fixed_words)
{
    if (!ctx || !context_words || !fixed_words) return fail(ctx, OG_ERR_INVALID_ARG, "ctx", "null context or pointer");
    (void)hipSetDevice(ctx->device);
    auto count = [&](const void *dev, uint64_t words, uint64_t *out) {
        std::vector<unsigned long long> h(words);
        hipError_t e = words ? hipMemcpyAsync(h.data(), dev, words * 8, hipMemcpyDeviceToHost, ctx->stream) : hipSuccess;
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        *out = (uint64_t)std::count_if(h.begin(), h.end(), [](unsigned long long w) { return w != 0; });
        return e;
    };
    hipError_t e = count(ctx->xcd_words, ctx->xcd_words ? ctx->xcd_word_count : 0, context_words);
    if (e == hipSuccess) e = count(ctx->noalloc_scratch, ctx->noalloc_scratch ? og::kNoAllocWordBytes / 8 : 0, fixed_words);
    return e == hipSuccess ? ok(ctx) : hip_status(ctx, e, "og_test_nonzero_words");
}

}  // extern "C"
