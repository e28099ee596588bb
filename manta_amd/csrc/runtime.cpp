// runtime.cpp -- implementation of the C ABI in include/manta_rocm.h.
//
// Host side of the rocm backend: argument validation with the reference's
// error conditions and wording, device memory, candidate binding, workspace
// management and the launch sequences of each entry point.  The reference
// counterpart is the cgo preamble and deviceRuntime of
// runtime/backends/cuda/native_linux.go; the semantic checks mirror
// runtime/backend/tensor_ops.go (scoreLayout :1499-1521, topKTensor
// :1523-1534, gatherTensor :794-877).
#include "manta_rocm.h"
#include "manta_mll.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <thread>
#include <vector>

#include "device_common.hpp"
#include "kernels.hpp"
#include "pack.hpp"
#include "runtime_internal.hpp"

using manta::QConst;
using manta::ScanArgs;

struct TimedLaunch {
    const char* name;
    hipEvent_t start;
    hipEvent_t stop;
};

struct MantaRocm {
    int device = 0;
    int cus = 256;  // compute units of the device (hipDeviceAttributeMultiprocessorCount)
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    // reference-semantics top-k: the scan's candidates and the finish's
    // verdicts, kept apart from ws (which the scans and the rescan use)
    void* ws_ref = nullptr;
    size_t ws_ref_bytes = 0;
    MantaRocmStats stats{};
    // first out-of-range gather index seen by a device gather (flag | index)
    unsigned long long* err_word = nullptr;
    bool gather_pending = false;
    // per-query tickets of the last-workgroup merge (zero between calls)
    uint32_t* tickets = nullptr;
    // per-kernel-family timing (manta_rocm_set_timing)
    bool timing = false;
    std::vector<TimedLaunch> pending;
    std::vector<hipEvent_t> event_pool;
    std::map<std::string, std::pair<uint64_t, double>> totals;
    // span timing (manta_rocm_span): events around a run of launches
    hipEvent_t span_ev[2] = {nullptr, nullptr};
    // candidate sets bound on this runtime and not yet unbound: destroy
    // releases their device memory and detaches them
    std::set<MantaRocmCandidates*> bound;
};

struct MantaRocmCandidates {
    MantaRocm* rt = nullptr;
    int format = 0;
    int64_t sets = 0, n = 0, d = 0;
    int pitch = 0;  // bytes per row in device memory
    int nb = 0;     // q4 blocks per row
    void* codes = nullptr;
    void* scales = nullptr;
    float* dnorm = nullptr;
    float* dd = nullptr;
    double* sqd = nullptr;  // [sets][n] sqrt of each row's f64 square-sum (reference cosine)
    float maxdn = 0.0f;     // max over rows of dnorm
    float maxdd = 0.0f;     // max over rows of dd
    // the quantized-query scans may rank rows for reference-semantics
    // top-k: every scale finite and zero or within [2^-60, 2^60] (the
    // scans' error bounds hold without underflow or overflow)
    bool ref_ranked = false;
    mutable size_t bytes = 0;
    bool scales_finite = false;  // every row / block scale is finite (the 512-query kernel needs it)
    bool scales_nonneg = false;  // q8: no row scale is below zero (the 512-query kernel's pre-filter needs it)
    // q4: int8 shadow for many-query top-k (built on first use): codes
    // [n][shadow_pitch], scales [2][n] (dot, cosine), error bounds
    mutable int shadow_state = 0;  // 0 not built, 1 built, -1 unavailable
    mutable int shadow_pitch = 0;
    mutable int8_t* shadow_codes = nullptr;
    mutable float* shadow_scales = nullptr;
    mutable manta::ShadowInfo* shadow_info = nullptr;
};

namespace {

constexpr int64_t kMaxDim = 1024;     // exactness bound of the int32 / f32 accumulators
constexpr int64_t kMaxDeviceK = 2048;  // reservoir capacity bound (LDS, cap <= 4096)
constexpr int64_t kTickets = 65536;    // last-workgroup tickets (queries / sequences per call)

char* dup_printf(const char* fmt, va_list ap) {
    va_list ap2;
    va_copy(ap2, ap);
    int n = vsnprintf(nullptr, 0, fmt, ap2);
    va_end(ap2);
    if (n < 0) return nullptr;
    char* out = (char*)malloc((size_t)n + 1);
    if (!out) return nullptr;
    vsnprintf(out, (size_t)n + 1, fmt, ap);
    return out;
}

int fail(char** err, int code, const char* fmt, ...) {
    if (err) {
        va_list ap;
        va_start(ap, fmt);
        *err = dup_printf(fmt, ap);
        va_end(ap);
    }
    return code;
}

int hip_fail(char** err, const char* what, hipError_t e) {
    return fail(err, MANTA_ROCM_ERROR, "%s: %s (%s)", what, hipGetErrorName(e),
                hipGetErrorString(e));
}

#define HIP_TRY(call, what)                                  \
    do {                                                     \
        hipError_t e_ = (call);                              \
        if (e_ != hipSuccess) return hip_fail(err, what, e_); \
    } while (0)

hipEvent_t pooled_event(MantaRocm* rt) {
    if (!rt->event_pool.empty()) {
        hipEvent_t e = rt->event_pool.back();
        rt->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Every kernel launch goes through here: counts it and, when timing is on,
// brackets it with events on the runtime's stream.
#define LAUNCH_TRY(call, what)                                                  \
    do {                                                                        \
        hipEvent_t ea_ = nullptr, eb_ = nullptr;                                \
        if (rt->timing) {                                                       \
            ea_ = pooled_event(rt);                                             \
            if (ea_) (void)hipEventRecord(ea_, rt->stream);                     \
        }                                                                       \
        HIP_TRY((call), what);                                                  \
        if (rt->timing && ea_) {                                                \
            eb_ = pooled_event(rt);                                             \
            if (eb_) {                                                          \
                (void)hipEventRecord(eb_, rt->stream);                          \
                rt->pending.push_back(TimedLaunch{what, ea_, eb_});             \
            } else {                                                            \
                rt->event_pool.push_back(ea_);                                  \
            }                                                                   \
        }                                                                       \
        rt->stats.kernel_launches++;                                            \
    } while (0)

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

int grow_buffer(MantaRocm* rt, void** buf, size_t* have, size_t bytes, char** err) {
    if (bytes <= *have) return MANTA_ROCM_OK;
    if (*buf) {
        HIP_TRY(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
        HIP_TRY(hipFree(*buf), "hipFree");
        *buf = nullptr;
        *have = 0;
    }
    size_t want = align_up(bytes, (size_t)1 << 20);
    HIP_TRY(hipMalloc(buf, want), "hipMalloc(workspace)");
    *have = want;
    rt->stats.workspace_bytes = rt->ws_bytes + rt->ws_ref_bytes;
    return MANTA_ROCM_OK;
}

int ensure_workspace(MantaRocm* rt, size_t bytes, char** err) {
    return grow_buffer(rt, &rt->ws, &rt->ws_bytes, bytes, err);
}

int ensure_ref_workspace(MantaRocm* rt, size_t bytes, char** err) {
    return grow_buffer(rt, &rt->ws_ref, &rt->ws_ref_bytes, bytes, err);
}

// `bytes` of device memory: from the caller's scratch when there is one
// (an error if it is exhausted), else the runtime workspace (grown on demand;
// one buffer per call path, so callers take it once).
int take_buffer(MantaRocm* rt, manta_rt::Scratch* sc, size_t bytes, void** out, char** err) {
    if (!sc) {
        int rc = ensure_workspace(rt, bytes + 256, err);
        if (rc) return rc;
        *out = rt->ws;
        return MANTA_ROCM_OK;
    }
    const size_t at = align_up(sc->used, 256);
    if (at + bytes > sc->bytes)
        return fail(err, MANTA_ROCM_UNSUPPORTED,
                    "score_topk_noalloc: the call needs more than the %zu bytes of scratch the allocation-free "
                    "path holds", sc->bytes);
    *out = sc->base + at;
    sc->used = at + bytes;
    return MANTA_ROCM_OK;
}

// Carve a workspace into aligned slices.
struct Carver {
    char* base;
    size_t off = 0;
    explicit Carver(void* b) : base((char*)b) {}
    template <class T>
    T* take(size_t count) {
        off = align_up(off, 256);
        T* p = (T*)(base + off);
        off += count * sizeof(T);
        return p;
    }
};

int cap_for_k(int64_t k) {
    int cap = 512;
    while (cap < k + 256) cap <<= 1;
    return cap;
}

// Row consts over many rows, spread over host threads.
template <class F>
void parallel_rows(int64_t rows, F f) {
    unsigned hw = std::thread::hardware_concurrency();
    int64_t nt = std::min<int64_t>(hw ? hw : 4, 16);
    if (rows < 65536) nt = 1;
    if (nt <= 1) {
        f(0, rows);
        return;
    }
    std::vector<std::thread> th;
    int64_t per = (rows + nt - 1) / nt;
    for (int64_t t = 0; t < nt; t++) {
        int64_t a = t * per, b = std::min(rows, a + per);
        if (a >= b) break;
        th.emplace_back([=] { f(a, b); });
    }
    for (auto& x : th) x.join();
}

int set_device(MantaRocm* rt, char** err) {
    HIP_TRY(hipSetDevice(rt->device), "hipSetDevice");
    return MANTA_ROCM_OK;
}

// Device gathers record their out-of-range index of lowest position
// (report_gather_error) instead of faulting; the next synchronizing call
// reports it with gatherTensor's wording (tensor_ops.go:804-806) and clears
// it.
int check_gather_error(MantaRocm* rt, char** err) {
    if (!rt->gather_pending) return MANTA_ROCM_OK;
    rt->gather_pending = false;
    unsigned long long w = 0;
    HIP_TRY(hipMemcpyAsync(&w, rt->err_word, sizeof(w), hipMemcpyDeviceToHost, rt->stream),
            "hipMemcpy(error word)");
    HIP_TRY(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
    if (w == 0) return MANTA_ROCM_OK;
    const unsigned long long zero = 0;
    HIP_TRY(hipMemcpyAsync(rt->err_word, &zero, sizeof(zero), hipMemcpyHostToDevice, rt->stream),
            "hipMemcpy(error word)");
    HIP_TRY(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
    return fail(err, MANTA_ROCM_ERROR, "gather index %d out of range", manta_rt::gather_error_index(w));
}

#define RT_CHECK(rt)                                                          \
    do {                                                                      \
        if (!(rt)) return fail(err, MANTA_ROCM_ERROR, "nil rocm runtime");    \
        int rc_ = set_device((rt), err);                                      \
        if (rc_) return rc_;                                                  \
    } while (0)

int free_candidates_memory(MantaRocmCandidates* c) {
    if (!c) return 0;
    if (c->codes) (void)hipFree(c->codes);
    if (c->scales) (void)hipFree(c->scales);
    if (c->dnorm) (void)hipFree(c->dnorm);
    if (c->dd) (void)hipFree(c->dd);
    if (c->sqd) (void)hipFree(c->sqd);
    c->sqd = nullptr;
    if (c->shadow_codes) (void)hipFree(c->shadow_codes);
    if (c->shadow_scales) (void)hipFree(c->shadow_scales);
    if (c->shadow_info) (void)hipFree(c->shadow_info);
    c->codes = c->scales = nullptr;
    c->dnorm = c->dd = nullptr;
    c->shadow_codes = nullptr;
    c->shadow_scales = nullptr;
    c->shadow_info = nullptr;
    return 0;
}

void set_row_maxima(MantaRocmCandidates* c, const std::vector<float>& dnorm, const std::vector<float>& dd) {
    float mn = 0.0f, md = 0.0f;
    for (size_t i = 0; i < dnorm.size(); i++) {
        mn = std::fmax(mn, dnorm[i]);
        md = std::fmax(md, dd[i]);
    }
    c->maxdn = mn;
    c->maxdd = md;
}

}  // namespace

extern "C" {

int manta_rocm_abi_version(void) { return MANTA_ROCM_ABI_VERSION; }

void manta_rocm_free_error(char* msg) { free(msg); }

int manta_rocm_device_count(int* out, char** err) {
    if (!out) return fail(err, MANTA_ROCM_ERROR, "nil output");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) {
        *out = 0;
        return MANTA_ROCM_OK;
    }
    if (e != hipSuccess) {
        *out = 0;
        return hip_fail(err, "hipGetDeviceCount", e);
    }
    *out = n;
    return MANTA_ROCM_OK;
}

int manta_rocm_create(int device, MantaRocm** out, char** err) {
    if (!out) return fail(err, MANTA_ROCM_ERROR, "nil output");
    *out = nullptr;
    int n = 0;
    int rc = manta_rocm_device_count(&n, err);
    if (rc) return rc;
    if (n == 0) return fail(err, MANTA_ROCM_UNSUPPORTED, "no ROCm device available");
    if (device < 0 || device >= n)
        return fail(err, MANTA_ROCM_ERROR, "rocm device %d out of range (%d devices)", device, n);
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(err, MANTA_ROCM_UNSUPPORTED, "device %d is %s; libmanta_rocm is built for gfx950",
                    device, prop.gcnArchName);
    HIP_TRY(hipSetDevice(device), "hipSetDevice");
    MantaRocm* rt = new MantaRocm();
    rt->device = device;
    hipError_t e = hipStreamCreateWithFlags(&rt->own_stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete rt;
        return hip_fail(err, "hipStreamCreate", e);
    }
    rt->stream = rt->own_stream;
    {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0)
            rt->cus = cus;
    }
    // the allocation-free entry point's scratch address on this device
    manta_rt::noalloc_init(device);
    e = hipMalloc((void**)&rt->err_word, sizeof(unsigned long long));
    if (e == hipSuccess) e = hipMemset(rt->err_word, 0, sizeof(unsigned long long));
    if (e == hipSuccess) e = hipMalloc((void**)&rt->tickets, kTickets * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(rt->tickets, 0, kTickets * sizeof(uint32_t));
    if (e != hipSuccess) {
        (void)hipStreamDestroy(rt->own_stream);
        delete rt;
        return hip_fail(err, "hipMalloc(error word)", e);
    }
    *out = rt;
    return MANTA_ROCM_OK;
}

void manta_rocm_destroy(MantaRocm* rt) {
    if (!rt) return;
    (void)hipSetDevice(rt->device);
    (void)hipStreamSynchronize(rt->stream);
    for (auto& t : rt->pending) {
        (void)hipEventDestroy(t.start);
        (void)hipEventDestroy(t.stop);
    }
    for (auto e : rt->event_pool) (void)hipEventDestroy(e);
    for (auto e : rt->span_ev)
        if (e) (void)hipEventDestroy(e);
    if (rt->ws) (void)hipFree(rt->ws);
    if (rt->ws_ref) (void)hipFree(rt->ws_ref);
    if (rt->err_word) (void)hipFree(rt->err_word);
    if (rt->tickets) (void)hipFree(rt->tickets);
    // candidate sets still bound: their device memory goes with the runtime,
    // their handles stay valid for manta_rocm_unbind (which then frees only
    // the handle)
    for (MantaRocmCandidates* c : rt->bound) {
        free_candidates_memory(c);
        c->rt = nullptr;
    }
    rt->bound.clear();
    if (rt->own_stream) (void)hipStreamDestroy(rt->own_stream);
    delete rt;
}

int manta_rocm_set_stream(MantaRocm* rt, void* hip_stream, char** err) {
    RT_CHECK(rt);
    HIP_TRY(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
    rt->stream = hip_stream ? (hipStream_t)hip_stream : rt->own_stream;
    return MANTA_ROCM_OK;
}

int manta_rocm_synchronize(MantaRocm* rt, char** err) {
    RT_CHECK(rt);
    HIP_TRY(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
    return check_gather_error(rt, err);
}

int manta_rocm_malloc(MantaRocm* rt, void** out_dev, size_t bytes, char** err) {
    RT_CHECK(rt);
    if (!out_dev) return fail(err, MANTA_ROCM_ERROR, "nil output");
    *out_dev = nullptr;
    HIP_TRY(hipMalloc(out_dev, bytes ? bytes : 1), "hipMalloc");
    return MANTA_ROCM_OK;
}

int manta_rocm_free(MantaRocm* rt, void* dev, char** err) {
    RT_CHECK(rt);
    if (!dev) return MANTA_ROCM_OK;
    HIP_TRY(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
    HIP_TRY(hipFree(dev), "hipFree");
    return MANTA_ROCM_OK;
}

int manta_rocm_upload(MantaRocm* rt, void* dst_dev, const void* src, size_t bytes, char** err) {
    RT_CHECK(rt);
    if (bytes == 0) return MANTA_ROCM_OK;
    if (!dst_dev || !src) return fail(err, MANTA_ROCM_ERROR, "nil upload pointer");
    HIP_TRY(hipMemcpyAsync(dst_dev, src, bytes, hipMemcpyHostToDevice, rt->stream),
            "hipMemcpyHtoD");
    HIP_TRY(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
    rt->stats.bytes_uploaded += bytes;
    return MANTA_ROCM_OK;
}

int manta_rocm_download(MantaRocm* rt, void* dst, const void* src_dev, size_t bytes, char** err) {
    RT_CHECK(rt);
    if (bytes == 0) return MANTA_ROCM_OK;
    if (!dst || !src_dev) return fail(err, MANTA_ROCM_ERROR, "nil download pointer");
    HIP_TRY(hipMemcpyAsync(dst, src_dev, bytes, hipMemcpyDeviceToHost, rt->stream),
            "hipMemcpyDtoH");
    HIP_TRY(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
    rt->stats.bytes_downloaded += bytes;
    return check_gather_error(rt, err);
}

int manta_rocm_set_timing(MantaRocm* rt, int on, char** err) {
    RT_CHECK(rt);
    rt->timing = on != 0;
    return MANTA_ROCM_OK;
}

int manta_rocm_timing(MantaRocm* rt, const char* name, uint64_t* count, double* total_ms, int reset,
                      char** err) {
    RT_CHECK(rt);
    HIP_TRY(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
    for (auto& t : rt->pending) {
        float ms = 0.0f;
        HIP_TRY(hipEventElapsedTime(&ms, t.start, t.stop), "hipEventElapsedTime");
        auto& tot = rt->totals[t.name];
        tot.first += 1;
        tot.second += ms;
        rt->event_pool.push_back(t.start);
        rt->event_pool.push_back(t.stop);
    }
    rt->pending.clear();
    uint64_t c = 0;
    double ms = 0.0;
    for (auto& kv : rt->totals) {
        if (name && kv.first != name) continue;
        c += kv.second.first;
        ms += kv.second.second;
    }
    if (count) *count = c;
    if (total_ms) *total_ms = ms;
    if (reset) rt->totals.clear();
    return MANTA_ROCM_OK;
}

int manta_rocm_span(MantaRocm* rt, int end, double* elapsed_ms, char** err) {
    RT_CHECK(rt);
    const int i = end ? 1 : 0;
    if (!rt->span_ev[i]) HIP_TRY(hipEventCreate(&rt->span_ev[i]), "hipEventCreate");
    HIP_TRY(hipEventRecord(rt->span_ev[i], rt->stream), "hipEventRecord");
    if (!end) return MANTA_ROCM_OK;
    if (!rt->span_ev[0]) return fail(err, MANTA_ROCM_ERROR, "span: no start mark");
    HIP_TRY(hipEventSynchronize(rt->span_ev[1]), "hipEventSynchronize");
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, rt->span_ev[0], rt->span_ev[1]), "hipEventElapsedTime");
    if (elapsed_ms) *elapsed_ms = ms;
    return MANTA_ROCM_OK;
}

int manta_rocm_stats(const MantaRocm* rt, MantaRocmStats* out) {
    if (!rt || !out) return MANTA_ROCM_ERROR;
    *out = rt->stats;
    return MANTA_ROCM_OK;
}

// ------------------------------------------------------------ packing

int manta_rocm_pack_q8_rows(const float* x, int64_t n, int64_t d, int8_t* codes, float* scales,
                            char** err) {
    if (n < 0 || d <= 0) return fail(err, MANTA_ROCM_ERROR, "pack_q8_rows: bad shape [%lld,%lld]",
                                     (long long)n, (long long)d);
    if (!x || !codes || !scales) return fail(err, MANTA_ROCM_ERROR, "pack_q8_rows: nil pointer");
    parallel_rows(n, [&](int64_t a, int64_t b) {
        for (int64_t r = a; r < b; r++) scales[r] = manta::pack_q8_row(x + r * d, d, codes + r * d);
    });
    return MANTA_ROCM_OK;
}

int manta_rocm_pack_q4_blocks(const float* x, int64_t n, int64_t d, uint8_t* packed,
                              uint16_t* scales, char** err) {
    if (n < 0 || d <= 0 || d % 32 != 0)
        return fail(err, MANTA_ROCM_ERROR,
                    "pack_q4_blocks: d must be a positive multiple of 32 (got %lld)", (long long)d);
    if (!x || !packed || !scales) return fail(err, MANTA_ROCM_ERROR, "pack_q4_blocks: nil pointer");
    parallel_rows(n, [&](int64_t a, int64_t b) {
        for (int64_t r = a; r < b; r++)
            manta::pack_q4_row(x + r * d, d, packed + r * (d / 2), scales + r * (d / 32));
    });
    return MANTA_ROCM_OK;
}

int manta_rocm_pack_grid(const float* x, int64_t n, int64_t d, int bits, int8_t* codes, float* scales, int* grid,
                         char** err) {
    if (n < 0 || d <= 0) return fail(err, MANTA_ROCM_ERROR, "pack_grid: bad shape [%lld,%lld]", (long long)n,
                                     (long long)d);
    if (bits != 8 && bits != 4) return fail(err, MANTA_ROCM_ERROR, "pack_grid: bits must be 8 or 4 (got %d)", bits);
    if (!x || !codes || !scales || !grid) return fail(err, MANTA_ROCM_ERROR, "pack_grid: nil pointer");
    const int levels = (1 << (bits - 1)) - 1;
    // one grid for the whole tensor (the reference's own)
    const float s = manta::grid_scale(x, n * d, levels, codes);
    if (s >= 0.0f) {
        for (int64_t r = 0; r < n; r++) scales[r] = s;
        *grid = 2;
        return MANTA_ROCM_OK;
    }
    // a grid per row (e.g. rows packed per row and dequantized)
    std::atomic<bool> rows_ok{true};  // shared by the workers: any row off its grid stops them all
    parallel_rows(n, [&](int64_t a, int64_t b) {
        for (int64_t r = a; r < b && rows_ok.load(std::memory_order_relaxed); r++) {
            const float sr = manta::grid_scale(x + r * d, d, levels, codes + r * d);
            if (sr < 0.0f) rows_ok.store(false, std::memory_order_relaxed);
            scales[r] = sr;
        }
    });
    if (rows_ok.load()) {
        *grid = 1;
        return MANTA_ROCM_OK;
    }
    // on no grid: re-quantized per row to int8 (lossy)
    parallel_rows(n, [&](int64_t a, int64_t b) {
        for (int64_t r = a; r < b; r++) scales[r] = manta::pack_q8_row(x + r * d, d, codes + r * d);
    });
    *grid = 0;
    return MANTA_ROCM_OK;
}

// ------------------------------------------------------------- binding

int manta_rocm_bind_q8_rows(MantaRocm* rt, const int8_t* codes, const float* scales, int64_t sets,
                            int64_t n, int64_t d, MantaRocmCandidates** out, char** err) {
    RT_CHECK(rt);
    if (!out) return fail(err, MANTA_ROCM_ERROR, "nil output");
    *out = nullptr;
    if (sets <= 0 || n <= 0 || d <= 0)
        return fail(err, MANTA_ROCM_ERROR, "bind_q8_rows: bad shape [%lld,%lld,%lld]",
                    (long long)sets, (long long)n, (long long)d);
    if (d > kMaxDim)
        return fail(err, MANTA_ROCM_UNSUPPORTED, "bind_q8_rows: d=%lld exceeds the device limit %lld",
                    (long long)d, (long long)kMaxDim);
    if (n >= ((int64_t)1 << 31))
        return fail(err, MANTA_ROCM_UNSUPPORTED, "bind_q8_rows: n=%lld exceeds int32 ids", (long long)n);
    if (!codes || !scales) return fail(err, MANTA_ROCM_ERROR, "bind_q8_rows: nil pointer");
    const int64_t rows = sets * n;
    const int pitch = (int)align_up((size_t)d, 16);
    std::vector<float> dnorm((size_t)rows), dd((size_t)rows);
    std::vector<double> sqd((size_t)rows);
    parallel_rows(rows, [&](int64_t a, int64_t b) {
        for (int64_t r = a; r < b; r++) {
            manta::q8_row_consts(codes + r * d, scales[r], d, &dnorm[(size_t)r], &dd[(size_t)r]);
            sqd[(size_t)r] = manta::q8_row_ref_norm(codes + r * d, scales[r], d);
        }
    });
    auto* c = new MantaRocmCandidates();
    c->rt = rt;
    c->format = MANTA_ROCM_Q8_ROWS;
    bool finite = true, ranked = true, nonneg = true;
    for (int64_t r = 0; r < rows; r++) {
        const float a = std::fabs(scales[r]);
        finite = finite && std::isfinite(scales[r]);
        ranked = ranked && (a == 0.0f || (a >= 0x1p-60f && a <= 0x1p60f));
        nonneg = nonneg && !(scales[r] < 0.0f);
    }
    c->scales_finite = finite;
    c->scales_nonneg = nonneg;
    c->ref_ranked = finite && ranked;
    set_row_maxima(c, dnorm, dd);
    c->sets = sets;
    c->n = n;
    c->d = d;
    c->pitch = pitch;
    c->bytes = (size_t)rows * pitch + (size_t)rows * 20;
    hipError_t e = hipMalloc(&c->codes, (size_t)rows * pitch);
    if (e == hipSuccess) e = hipMalloc(&c->scales, (size_t)rows * 4);
    if (e == hipSuccess) e = hipMalloc((void**)&c->dnorm, (size_t)rows * 4);
    if (e == hipSuccess) e = hipMalloc((void**)&c->dd, (size_t)rows * 4);
    if (e == hipSuccess) e = hipMalloc((void**)&c->sqd, (size_t)rows * 8);
    if (e == hipSuccess) {
        if (pitch == d) {
            e = hipMemcpy(c->codes, codes, (size_t)rows * d, hipMemcpyHostToDevice);
        } else {
            std::vector<int8_t> tmp((size_t)rows * pitch, 0);
            for (int64_t r = 0; r < rows; r++) std::memcpy(&tmp[(size_t)(r * pitch)], codes + r * d, (size_t)d);
            e = hipMemcpy(c->codes, tmp.data(), tmp.size(), hipMemcpyHostToDevice);
        }
    }
    if (e == hipSuccess) e = hipMemcpy(c->scales, scales, (size_t)rows * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(c->dnorm, dnorm.data(), (size_t)rows * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(c->dd, dd.data(), (size_t)rows * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(c->sqd, sqd.data(), (size_t)rows * 8, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        free_candidates_memory(c);
        delete c;
        return hip_fail(err, "bind_q8_rows", e);
    }
    rt->stats.bytes_uploaded += c->bytes;
    rt->stats.candidate_bytes += c->bytes;
    rt->bound.insert(c);
    *out = c;
    return MANTA_ROCM_OK;
}

int manta_rocm_bind_packed(MantaRocm* rt, const MantaMll* container, MantaRocmCandidates** out, char** err) {
    RT_CHECK(rt);
    if (!out) return fail(err, MANTA_ROCM_ERROR, "nil output");
    *out = nullptr;
    int dtype = 0;
    uint64_t rows = 0;
    uint32_t dim = 0;
    const void *codes = nullptr, *scales = nullptr;
    int rc = manta_mll_packed_info(container, &dtype, &rows, &dim, &codes, &scales, nullptr, err);
    if (rc) return rc;
    if (dtype == MANTA_ROCM_Q8_ROWS)
        return manta_rocm_bind_q8_rows(rt, (const int8_t*)codes, (const float*)scales, 1, (int64_t)rows,
                                       (int64_t)dim, out, err);
    return manta_rocm_bind_q4_blocks(rt, (const uint8_t*)codes, (const uint16_t*)scales, 1, (int64_t)rows,
                                     (int64_t)dim, out, err);
}

int manta_rocm_bind_q4_blocks(MantaRocm* rt, const uint8_t* packed, const uint16_t* scales,
                              int64_t sets, int64_t n, int64_t d, MantaRocmCandidates** out,
                              char** err) {
    RT_CHECK(rt);
    if (!out) return fail(err, MANTA_ROCM_ERROR, "nil output");
    *out = nullptr;
    if (sets <= 0 || n <= 0 || d <= 0)
        return fail(err, MANTA_ROCM_ERROR, "bind_q4_blocks: bad shape [%lld,%lld,%lld]",
                    (long long)sets, (long long)n, (long long)d);
    if (d % 32 != 0)
        return fail(err, MANTA_ROCM_ERROR, "bind_q4_blocks: d must be a multiple of 32 (got %lld)",
                    (long long)d);
    if (d > kMaxDim)
        return fail(err, MANTA_ROCM_UNSUPPORTED, "bind_q4_blocks: d=%lld exceeds the device limit %lld",
                    (long long)d, (long long)kMaxDim);
    if (n >= ((int64_t)1 << 31))
        return fail(err, MANTA_ROCM_UNSUPPORTED, "bind_q4_blocks: n=%lld exceeds int32 ids", (long long)n);
    if (!packed || !scales) return fail(err, MANTA_ROCM_ERROR, "bind_q4_blocks: nil pointer");
    const int64_t rows = sets * n;
    const int pitch = (int)(d / 2);
    const int nb = (int)(d / 32);
    std::vector<float> dnorm((size_t)rows), dd((size_t)rows);
    std::vector<double> sqd((size_t)rows);
    parallel_rows(rows, [&](int64_t a, int64_t b) {
        for (int64_t r = a; r < b; r++) {
            manta::q4_row_consts(packed + r * pitch, scales + r * nb, d, &dnorm[(size_t)r], &dd[(size_t)r]);
            sqd[(size_t)r] = manta::q4_row_ref_norm(packed + r * pitch, scales + r * nb, d);
        }
    });
    auto* c = new MantaRocmCandidates();
    c->rt = rt;
    c->format = MANTA_ROCM_Q4_BLOCKS;
    bool finite = true;  // f16 exponent field below all-ones
    for (int64_t i = 0; i < rows * nb && finite; i++) finite = (scales[i] & 0x7C00u) != 0x7C00u;
    c->scales_finite = finite;
    c->ref_ranked = finite;  // finite f16 scales are within [2^-24, 2^16]
    set_row_maxima(c, dnorm, dd);
    c->sets = sets;
    c->n = n;
    c->d = d;
    c->pitch = pitch;
    c->nb = nb;
    c->bytes = (size_t)rows * (pitch + nb * 2 + 16);
    hipError_t e = hipMalloc(&c->codes, (size_t)rows * pitch);
    if (e == hipSuccess) e = hipMalloc(&c->scales, (size_t)rows * nb * 2);
    if (e == hipSuccess) e = hipMalloc((void**)&c->dnorm, (size_t)rows * 4);
    if (e == hipSuccess) e = hipMalloc((void**)&c->dd, (size_t)rows * 4);
    if (e == hipSuccess) e = hipMalloc((void**)&c->sqd, (size_t)rows * 8);
    if (e == hipSuccess) e = hipMemcpy(c->codes, packed, (size_t)rows * pitch, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(c->scales, scales, (size_t)rows * nb * 2, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(c->dnorm, dnorm.data(), (size_t)rows * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(c->dd, dd.data(), (size_t)rows * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(c->sqd, sqd.data(), (size_t)rows * 8, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        free_candidates_memory(c);
        delete c;
        return hip_fail(err, "bind_q4_blocks", e);
    }
    rt->stats.bytes_uploaded += c->bytes;
    rt->stats.candidate_bytes += c->bytes;
    rt->bound.insert(c);
    *out = c;
    return MANTA_ROCM_OK;
}

void manta_rocm_unbind(MantaRocmCandidates* cands) {
    if (!cands) return;
    if (cands->rt) {
        (void)hipSetDevice(cands->rt->device);
        (void)hipStreamSynchronize(cands->rt->stream);
        cands->rt->stats.candidate_bytes -= std::min<uint64_t>(cands->rt->stats.candidate_bytes, cands->bytes);
        cands->rt->bound.erase(cands);
        free_candidates_memory(cands);
    }
    // (a set whose runtime was destroyed first has no device memory left)
    delete cands;
}

int manta_rocm_candidates_info(const MantaRocmCandidates* c, int* format, int64_t* sets, int64_t* n,
                               int64_t* d) {
    if (!c) return MANTA_ROCM_ERROR;
    if (format) *format = c->format;
    if (sets) *sets = c->sets;
    if (n) *n = c->n;
    if (d) *d = c->d;
    return MANTA_ROCM_OK;
}

// ------------------------------------------------------------- scoring

namespace {

ScanArgs scan_args(const MantaRocmCandidates* c, const uint16_t* q) {
    ScanArgs a{};
    a.codes = (const int8_t*)c->codes;
    a.scales = c->scales;
    a.dnorm = c->dnorm;
    a.dd = c->dd;
    a.n = c->n;
    a.pitch = c->pitch;
    a.nb = c->nb;
    a.d = (int)c->d;
    a.set_stride = (c->sets == 1) ? 0 : c->n;
    a.queries = q;
    return a;
}

// A score op as the ABI takes it: the builtin (dot / cosine / l2_distance)
// and the MANTA_ROCM_QUANTIZED_QUERY flag.  scan: the device op of the
// quantized-query scans (q8 dot: E8 codes when the caller asked for them,
// else E16; every other op E16); ref: the reference arithmetic's.
struct ScoreOp {
    int op = 0;
    bool quant = false;
    int scan = 0;
    int ref = 0;
};

ScoreOp parse_op(const MantaRocmCandidates* c, int op_in) {
    ScoreOp so;
    so.op = op_in & ~MANTA_ROCM_QUANTIZED_QUERY;
    so.quant = (op_in & MANTA_ROCM_QUANTIZED_QUERY) != 0;
    so.ref = so.op == MANTA_ROCM_DOT ? manta::OP_DOT : (so.op == MANTA_ROCM_COSINE ? manta::OP_COSINE : manta::OP_L2);
    so.scan = so.ref;
    if (so.op == MANTA_ROCM_DOT && c->format == MANTA_ROCM_Q8_ROWS && !so.quant) so.scan = manta::OP_DOT16;
    return so;
}

int check_score_args(const MantaRocmCandidates* c, int op_in, const void* q, int64_t nq, char** err) {
    if (!c) return fail(err, MANTA_ROCM_ERROR, "nil score input");
    const int op = op_in & ~MANTA_ROCM_QUANTIZED_QUERY;
    if (op < MANTA_ROCM_DOT || op > MANTA_ROCM_L2_DISTANCE)
        return fail(err, MANTA_ROCM_ERROR, "unknown score op %d", op_in);
    if (!q) return fail(err, MANTA_ROCM_ERROR, "nil score input");
    if (nq <= 0) return fail(err, MANTA_ROCM_ERROR, "score expects at least one query");
    if (c->sets != 1 && c->sets != nq)
        return fail(err, MANTA_ROCM_ERROR, "score mismatch [%lld,%lld] x [%lld,%lld,%lld]", (long long)nq,
                    (long long)c->d, (long long)c->sets, (long long)c->n, (long long)c->d);
    if (nq > 65535) return fail(err, MANTA_ROCM_UNSUPPORTED, "more than 65535 queries in one call");
    if (c->d > manta::kMaxQueryDim)
        return fail(err, MANTA_ROCM_UNSUPPORTED, "query length %lld beyond the device path", (long long)c->d);
    return MANTA_ROCM_OK;
}

// Rounds of 256 rows per scan workgroup, for about `wgs` workgroups in all,
// so each streams a long contiguous range and the per-workgroup prologue and
// top-k publication are paid rarely.  The fused top-k takes one workgroup
// per CU (C0's 32 problems: 82.3 us a launch against 85.1 with two per CU,
// 97.6 with one per two CUs and 99.2 with 1.25 per CU); the score matrix
// keeps two per CU.
int choose_rounds(int64_t tiles, int64_t nq, int64_t wgs) {
    int64_t r = (tiles * nq + wgs - 1) / wgs;
    // small calls are latency-bound: two rounds halve the parts the last
    // workgroup merges (one 65536 x 256 query, with the lists filled and
    // merged by rank: 13.3 us a call against 15.8 with one round and 14.1
    // with four)
    if (r < 2 && tiles >= 4) r = 2;
    return (int)std::max<int64_t>(1, std::min<int64_t>(64, r));
}

// Launch shape of a streaming top-k (one query per blockIdx.y): `parts`
// workgroups of `rounds` x 256 rows per query, and the LDS reservoir.  A
// reservoir that holds every row of the workgroup needs no compaction (and
// no barrier) between rounds.
struct StreamTopk {
    int rounds = 1;
    int64_t parts = 1;
    int cap = 0;
    int mid_compact = 1;
    int lds_keys = 0;
};

StreamTopk stream_topk_shape(const MantaRocmCandidates* c, int64_t nq, int64_t k, int rounds) {
    StreamTopk st;
    const int64_t tiles = (c->n + 255) / 256;
    st.rounds = rounds;
    st.parts = (tiles + rounds - 1) / rounds;
    st.cap = cap_for_k(k);
    if (k + (int64_t)rounds * 256 <= manta::kMaxCapKeys) {
        st.cap = cap_for_k(k + (int64_t)(rounds - 1) * 256);
        st.mid_compact = 0;
    }
    // the merge loads all parts at once when they fit in LDS (<= 4096 keys)
    st.lds_keys = (int)std::max<int64_t>(st.cap, st.parts * k <= manta::kMaxCapKeys ? st.parts * k : 0);
    (void)nq;
    return st;
}

// Streaming top-k arguments; the parts' keys go to `partial` ([nq][parts][k]).
ScanArgs stream_topk_args(const MantaRocmCandidates* c, const uint16_t* q, const StreamTopk& st, int64_t k,
                          int order, int32_t* out_ids, float* out_scores, uint64_t* partial, uint32_t* tickets) {
    ScanArgs a = scan_args(c, q);
    a.mid_compact = st.mid_compact;
    a.rounds = st.rounds;
    a.partial = partial;
    a.tickets = tickets;
    a.out_ids = out_ids;
    a.out_topk_scores = out_scores;
    a.k = (int)k;
    a.cap = st.cap;
    a.lds_keys = st.lds_keys;
    a.smallest = order == MANTA_ROCM_SMALLEST;
    return a;
}

int launch_scan(MantaRocm* rt, const MantaRocmCandidates* c, int op, const ScanArgs& a, dim3 grid,
                size_t lds, char** err) {
    if (c->format == MANTA_ROCM_Q8_ROWS)
        LAUNCH_TRY(manta::launch_q8_scan(op, a, grid, lds, rt->stream), "q8_scan");
    else
        LAUNCH_TRY(manta::launch_q4_scan(op, a, grid, lds, rt->stream), "q4_scan");
    return MANTA_ROCM_OK;
}

}  // namespace

}  // extern "C"

namespace {

// Multi-query plan: many queries against one shared q8 matrix go to the
// matrix-core kernels (kernels_mq.hip); everything else streams one query per
// workgroup.  Top-k runs in passes over growing row prefixes: pass 0 keeps
// every key of its rows, and each later pass starts from the k-th best key
// of all earlier rows, so only a few times k keys per query survive a pass.
struct MqPass {
    int64_t begin = 0;
    int64_t end = 0;
    int64_t rows_per_wg = 0;
    int R = 0;
    int select_threads = 256;
};

struct MqPlan {
    bool use = false;
    bool q4 = false;     // q4 blocks (kernels_mq4.hip, or the shadow scan), else q8 rows
    bool shadow = false; // q4 through its int8 shadow on the 512-query kernel
    manta::MqShape sh;
    int groups = 0;
    int rc = 0;          // region capacity (keys per query and workgroup)
    int rmax = 0;        // largest grid.x over the passes
    size_t lds = 0;
    std::vector<MqPass> passes;
};

constexpr int kMqWorkgroups = 512;     // two 256-thread workgroups per CU of a 256-CU MI355X
constexpr int kMq8Workgroups = 256;    // one 512-thread workgroup per CU
constexpr int64_t kMqSelectKeys = 16384;  // LDS keys of the select kernel

MqPass mq_pass(int64_t begin, int64_t end, int chunk, int groups, int64_t max_rows_per_wg, int wgs) {
    MqPass p;
    p.begin = begin;
    p.end = end;
    const int64_t chunks = (end - begin + chunk - 1) / chunk;
    int64_t R = std::max<int64_t>(1, std::min<int64_t>(chunks, std::max(1, wgs / groups)));
    int64_t cpw = (chunks + R - 1) / R;
    if (max_rows_per_wg > 0) cpw = std::max<int64_t>(1, std::min<int64_t>(cpw, max_rows_per_wg / chunk));
    p.rows_per_wg = cpw * chunk;
    p.R = (int)((chunks + cpw - 1) / cpw);
    return p;
}

// Region capacity of the 512-query kernel for k; its free chunk tile must
// hold a region's pairs and keys when it compacts one.
int mq8_rc(int64_t k) { return (int)(((2 * k + 2 * 64 + 64) + 63) / 64 * 64); }

bool mq8_fits(int pitch, int64_t k) {
    return manta::mq8_supported(pitch) && (size_t)mq8_rc(k) * 16 <= (size_t)manta::mq8_shape(pitch, 1, false).tile;
}

// q4 cosine / dot top-k with at least 256 queries goes through the int8
// shadow (built on first use).
bool q4_shadow_wanted(const MantaRocmCandidates* c, int dop, int64_t nq, int64_t k) {
    return c->format == MANTA_ROCM_Q4_BLOCKS && c->sets == 1 && (dop == manta::OP_COSINE || dop == manta::OP_DOT) &&
           nq >= 256 && c->d <= 384 && c->scales_finite && mq8_fits((int)align_up((size_t)c->d, 128), k);
}

// Build the int8 shadow of a q4 matrix on its first many-query top-k call
// (stream-ordered kernels; the allocation is the only host-side work).  If
// the memory is not there the q4 kernels keep serving such calls.
void ensure_q4_shadow(MantaRocm* rt, const MantaRocmCandidates* c) {
    if (c->shadow_state != 0) return;
    const int sp = (int)align_up((size_t)c->d, 128);
    const int64_t n = c->n;
    int8_t* codes = nullptr;
    float* sc = nullptr;
    manta::ShadowInfo* info = nullptr;
    hipError_t e = hipMalloc(&codes, (size_t)n * sp);
    if (e == hipSuccess) e = hipMalloc(&sc, (size_t)n * 8);
    if (e == hipSuccess) e = hipMalloc(&info, sizeof(manta::ShadowInfo));
    if (e == hipSuccess) e = manta::launch_shadow_info_clear(info, rt->stream);
    if (e == hipSuccess)
        e = manta::launch_q4_shadow_build((const uint8_t*)c->codes, (const uint16_t*)c->scales, c->dnorm, n,
                                          (int)c->d, sp, codes, sc, sc + n, info, rt->stream);
    if (e != hipSuccess) {
        if (codes) (void)hipFree(codes);
        if (sc) (void)hipFree(sc);
        if (info) (void)hipFree(info);
        (void)hipGetLastError();
        c->shadow_state = -1;
        return;
    }
    c->shadow_codes = codes;
    c->shadow_scales = sc;
    c->shadow_info = info;
    c->shadow_pitch = sp;
    c->shadow_state = 1;
    const size_t extra = (size_t)n * sp + (size_t)n * 8 + sizeof(manta::ShadowInfo);
    c->bytes += extra;
    rt->stats.candidate_bytes += extra;
}

MqPlan mq_plan(const MantaRocmCandidates* c, int dop, int64_t nq, int64_t k, bool topk) {
    MqPlan p;
    if (c->sets != 1 || nq < 8) return p;
    // the 16x16x64 kernel: 512-query groups, or 256 with the rows of a chunk
    // split over two wave groups
    const int ws8 = nq >= 512 ? 1 : 2;
    if (c->format == MANTA_ROCM_Q8_ROWS) {
        if (topk && dop == manta::OP_DOT && nq >= 256 && c->scales_finite && c->scales_nonneg &&
            mq8_fits(c->pitch, k)) {
            p.sh = manta::mq8_shape(c->pitch, ws8, false);
        } else {
            if (c->pitch % 32 != 0 || !manta::mq_supported_ks(c->pitch / 32)) return p;
            p.sh = manta::mq_shape(dop, c->pitch / 32, nq);
        }
    } else {
        p.q4 = true;
        if (topk && c->shadow_state == 1 && q4_shadow_wanted(c, dop, nq, k)) {
            p.shadow = true;
            p.sh = manta::mq8_shape(c->shadow_pitch, ws8, true);
        } else {
            if (!manta::mq4_supported_nb(c->nb)) return p;
            p.sh = manta::mq4_shape(dop, c->nb, nq);
        }
    }
    p.groups = (int)((nq + p.sh.qg - 1) / p.sh.qg);
    if (p.groups > 65535) return p;
    const int chunk = p.sh.chunk;
    const int wgs = p.sh.kind == 1 ? kMq8Workgroups : kMqWorkgroups;
    if (!topk) {
        p.passes.push_back(mq_pass(0, c->n, chunk, p.groups, 0, wgs));
        p.rmax = p.passes[0].R;
        p.lds = (size_t)p.sh.tile_bytes;
        p.use = true;
        return p;
    }
    // region: the best k after a compaction plus one chunk of appends, with
    // slack so a compaction frees at least k slots (the 512-query kernel
    // needs rc >= k + 2.5 chunks: true for its chunks of 64 or 128 rows)
    p.rc = (int)(((2 * k + 2 * chunk + 64) + 63) / 64 * 64);
    p.lds = (size_t)p.sh.tile_bytes +
            (p.sh.kind == 0 && (size_t)p.rc * 8 > (size_t)p.sh.tile ? (size_t)p.rc * 8 : 0);
    // pass 0: everything is kept, so a workgroup takes at most rc - 2*chunk rows
    int64_t s = std::min<int64_t>(c->n, std::max<int64_t>(8 * k, 4096));
    p.passes.push_back(mq_pass(0, s, chunk, p.groups, p.rc - 2 * chunk, wgs));
    p.passes.back().select_threads = manta::mq_select_threads(s);
    // shadow pairs are rescored by the select: 512 threads keep many row
    // loads in flight within the register budget
    if (p.shadow) p.passes.back().select_threads = 512;
    if (s < c->n) {
        // later passes grow the prefix by g: about k*g keys per query reach
        // the select.  Fewest passes the select's buffer allows, then the
        // smallest g that still needs no more of them.
        const double span = (double)c->n / (double)s;
        const double gmax = std::max(4.0, (double)kMqSelectKeys / (double)k);
        int npass = std::max(1, (int)std::ceil(std::log(span) / std::log(gmax) - 1e-9));
        // the 512-query kernel appends about k*(g-1) pairs per query and
        // pass, each an exact test and an LDS atomic in the scan: keep g
        // near 4.5 (measured on 1024 queries over 1024x the first pass's
        // rows: 5 passes beat 3 by 4% of the step, 6 and 7 lose to 5 on the
        // selects)
        if (p.sh.kind == 1 && !p.shadow)
            npass = std::max(npass, (int)std::ceil(std::log(span) / std::log(4.5) - 1e-9));
        // shadow pairs: every pair the select keeps is rescored from a random
        // row, so fewer, larger passes win as long as a pass's pairs (about
        // 4*k*g with the margins) fit the 512-thread select's 8K-key buffer,
        // which is what lets it prune before rescoring
        if (p.shadow) {
            const double gs = std::max(4.0, (8192.0 - (double)k) / (4.0 * (double)k));
            npass = std::max(1, (int)std::ceil(std::log(span) / std::log(gs) - 1e-9));
        }
        double g = std::pow(span, 1.0 / npass);
        // ... except its first growth pass, which grows the prefix by 16: over
        // so few rows the extra appends cost less than a pass and a select of
        // their own (1024 queries over 4M rows: 4,096 rows, then x16 and
        // three times x4 -- five passes instead of six -- measured 1,422 ->
        // 1,400 us a call; x8 gained nothing, x64 lost 35 us)
        double g0 = g;
        const double gfirst = std::min(16.0, gmax);
        if (p.sh.kind == 1 && !p.shadow && span > gfirst * 4.5) {
            const double rest = span / gfirst;
            npass = 1 + (int)std::ceil(std::log(rest) / std::log(4.5) - 1e-9);
            g0 = gfirst;
            g = std::pow(rest, 1.0 / (npass - 1));
        }
        for (int i = 0; i < npass; i++) {
            const double gi = i == 0 ? g0 : g;
            const int64_t e = i + 1 == npass ? c->n : std::min<int64_t>(c->n, (int64_t)std::ceil(s * gi));
            if (e <= s) continue;
            p.passes.push_back(mq_pass(s, e, chunk, p.groups, 0, wgs));
            // (shadow pairs: the margins let a few times more through)
            p.passes.back().select_threads =
                p.shadow ? 512 : manta::mq_select_threads(k + (int64_t)(k * (gi - 1.0) * 1.5));
            s = e;
        }
    }
    for (const MqPass& ps : p.passes) p.rmax = std::max(p.rmax, ps.R);
    // the kernels index regions with 32-bit offsets
    if ((int64_t)nq * p.rmax * p.rc >= ((int64_t)1 << 31)) return p;
    p.use = true;
    return p;
}

hipError_t launch_mq_pass(const MqPlan& p, int dop, const manta::MqArgs& a, int R, hipStream_t s) {
    const dim3 grid((unsigned)R, (unsigned)p.groups);
    if (p.sh.kind == 1) return manta::launch_mq8_scan(p.sh, a, grid, p.lds, s);
    return p.q4 ? manta::launch_mq4_scan(dop, p.sh, a, grid, p.lds, s) : manta::launch_mq_scan(dop, p.sh, a, grid, p.lds, s);
}

// Encode queries to the global digit planes, then run the multi-query passes.
int run_mq(MantaRocm* rt, const MantaRocmCandidates* c, int dop, int order, const uint16_t* q, int64_t nq,
           int64_t k, const MqPlan& p, float* out_scores, int32_t* out_ids, float* out_topk_scores,
           char** err, bool any_order = false) {
    // query planes: E8 codes or E16 digits, one row per query, as wide as a
    // q8 row (pitch) or a q4 row in elements (d); the shadow scan's E8
    // codes are as wide as a shadow row, its E16 planes [nq][d]
    const int width = p.shadow ? c->shadow_pitch : (p.q4 ? (int)c->d : c->pitch);
    const size_t plane = (size_t)nq * width;
    const bool topk = out_scores == nullptr;
    const size_t regions = topk ? (size_t)nq * p.rmax * p.rc : 0;
    const size_t counts = topk ? (size_t)nq * p.rmax : 0;
    size_t need = 3 * (plane + 256) + (size_t)nq * sizeof(QConst) + 256 + (size_t)nq * 12 + 512 +
                  (size_t)nq * (size_t)k * 8 + 256 + regions * 8 + 256 + counts * 4 + 256 + (size_t)nq * 8 + 256;
    int rc = ensure_workspace(rt, need, err);
    if (rc) return rc;
    Carver cv(rt->ws);
    int8_t* c8 = cv.take<int8_t>(plane);
    int8_t* hi = cv.take<int8_t>(plane);
    int8_t* lo = cv.take<int8_t>(plane);
    QConst* qc = cv.take<QConst>((size_t)nq);
    uint64_t* tau = cv.take<uint64_t>((size_t)nq);
    int* bcnt = cv.take<int>((size_t)nq);
    uint64_t* best = cv.take<uint64_t>(topk ? (size_t)nq * k : 1);
    uint64_t* reg = cv.take<uint64_t>(regions ? regions : 1);
    int* cnt = cv.take<int>(counts ? counts : 1);
    float* qb = cv.take<float>((size_t)nq * 2);
    if (p.shadow) {
        LAUNCH_TRY(manta::launch_query_encode_shadow(q, (int)nq, (int)c->d, width, dop, c->shadow_info, c8, hi, lo,
                                                     qc, qb, topk ? tau : nullptr, topk ? bcnt : nullptr, rt->stream),
                   "query_encode");
    } else {
        const int e16 = p.q4 ? 2 : (dop != manta::OP_DOT ? 1 : 0);
        LAUNCH_TRY(manta::launch_query_encode(q, (int)nq, (int)c->d, width, e16, c8, hi, lo, qc,
                                              topk ? tau : nullptr, topk ? bcnt : nullptr, rt->stream),
                   "query_encode");
    }
    manta::MqArgs a{};
    a.codes = p.shadow ? c->shadow_codes : (const int8_t*)c->codes;
    a.scales = p.shadow ? c->shadow_scales + (dop == manta::OP_COSINE ? c->n : 0) : (const float*)c->scales;
    a.dnorm = c->dnorm;
    a.dd = c->dd;
    a.n = c->n;
    a.pitch = p.shadow ? c->shadow_pitch : c->pitch;
    a.qbound = qb;
    a.q4codes = (const uint8_t*)c->codes;
    a.q4scales = (const uint16_t*)c->scales;
    a.d = (int)c->d;
    a.op = dop;
    a.nq = (int)nq;
    a.qc8 = c8;
    a.qhi = hi;
    a.qlo = lo;
    a.qconst = qc;
    a.tau = tau;
    a.regions = reg;
    a.counts = cnt;
    a.rc = p.rc;
    a.k = (int)k;
    a.out_scores = out_scores;
    a.smallest = order == MANTA_ROCM_SMALLEST;
    if (!topk) {
        const MqPass& ps = p.passes[0];
        a.row_begin = ps.begin;
        a.row_end = ps.end;
        a.rows_per_wg = ps.rows_per_wg;
        a.R = ps.R;
        LAUNCH_TRY(launch_mq_pass(p, dop, a, ps.R, rt->stream), "mq_scan");
        return MANTA_ROCM_OK;
    }
    // (tau and bcnt were reset by the query encoding above)
    manta::MqSelectArgs sa{};
    sa.regions = reg;
    sa.counts = cnt;
    sa.rc = p.rc;
    sa.best = best;
    sa.bcnt = bcnt;
    sa.tau = tau;
    sa.k = (int)k;
    sa.nq = (int)nq;
    sa.smallest = a.smallest;
    // the 512-query kernel's regions hold (pre-score, row) pairs: q8 dot
    // keys follow from the pre-score, shadow pairs are rescored exactly
    sa.pairs = p.sh.kind == 1 ? (p.shadow ? 2 : 1) : 0;
    sa.qconst = qc;
    sa.q4codes = (const uint8_t*)c->codes;
    sa.q4scales = (const uint16_t*)c->scales;
    sa.dnorm = c->dnorm;
    sa.dd = c->dd;
    sa.qhi = hi;
    sa.qlo = lo;
    sa.qbound = qb;
    sa.d = (int)c->d;
    sa.op = dop;
    sa.unsorted = any_order ? 1 : 0;
    for (size_t i = 0; i < p.passes.size(); i++) {
        const MqPass& ps = p.passes[i];
        a.row_begin = ps.begin;
        a.row_end = ps.end;
        a.rows_per_wg = ps.rows_per_wg;
        a.R = ps.R;
        // the first pass of the 512-query kernel keeps every pair: its
        // workgroups take at most rc - 2*chunk rows, one slot per row
        a.keep_all = i == 0 && p.sh.kind == 1 ? 1 : 0;
        LAUNCH_TRY(launch_mq_pass(p, dop, a, ps.R, rt->stream), "mq_scan");
        sa.R = ps.R;
        sa.uniform = a.keep_all ? (int)ps.rows_per_wg : 0;
        const bool last = i + 1 == p.passes.size();
        sa.out_ids = last ? out_ids : nullptr;
        sa.out_scores = last ? out_topk_scores : nullptr;
        LAUNCH_TRY(manta::launch_mq_select(sa, ps.select_threads, rt->stream), "mq_select");
    }
    return MANTA_ROCM_OK;
}

}  // namespace

extern "C" {

int manta_rocm_score(MantaRocm* rt, const MantaRocmCandidates* c, int op, const uint16_t* q,
                     int64_t nq, float* out, char** err) {
    RT_CHECK(rt);
    int rc = check_score_args(c, op, q, nq, err);
    if (rc) return rc;
    if (!out) return fail(err, MANTA_ROCM_ERROR, "nil score output");
    const ScoreOp so = parse_op(c, op);
    const int64_t tiles = (c->n + 255) / 256;
    if (!so.quant) {
        // the reference arithmetic for every (query, row)
        ScanArgs a = scan_args(c, q);
        a.rounds = (int)std::max<int64_t>(1, std::min<int64_t>(16, tiles * nq / 2048));
        a.out_scores = out;
        const int64_t parts = (tiles + a.rounds - 1) / a.rounds;
        LAUNCH_TRY(manta::launch_ref_scan(c->format == MANTA_ROCM_Q8_ROWS ? 8 : 4, so.ref, a, (int)nq, c->sqd,
                                          nullptr, nullptr, dim3((unsigned)parts, (unsigned)nq), 0, rt->stream),
                   "ref_scan");
        return MANTA_ROCM_OK;
    }
    const MqPlan plan = mq_plan(c, so.scan, nq, 0, false);
    if (plan.use) return run_mq(rt, c, so.scan, MANTA_ROCM_LARGEST, q, nq, 0, plan, out, nullptr, nullptr, err);
    ScanArgs a = scan_args(c, q);
    a.rounds = choose_rounds(tiles, nq, 512);
    a.out_scores = out;
    const int64_t parts = (tiles + a.rounds - 1) / a.rounds;
    return launch_scan(rt, c, so.scan, a, dim3((unsigned)parts, (unsigned)nq), 0, err);
}

}  // extern "C"

namespace {

// Top-k of the quantized-query scan scores (device op dop): the
// multi-query passes, or the streaming scan with its fused top-k.  With a
// caller's scratch (sc) the call allocates nothing: the streaming scan only,
// its keys and tickets in sc.
// any_order: the caller re-sorts the k rows (the reference finish), so the
// multi-query passes may return them in any order with the k-th best last.
int scan_topk(MantaRocm* rt, const MantaRocmCandidates* c, int dop, int order, const uint16_t* q, int64_t nq,
              int64_t k, int32_t* out_ids, float* out_scores, int64_t* out_acc, manta_rt::Scratch* sc, char** err,
              bool any_order = false) {
    if (!sc && q4_shadow_wanted(c, dop, nq, k)) ensure_q4_shadow(rt, c);
    const MqPlan plan = sc ? MqPlan() : mq_plan(c, dop, nq, k, true);
    const int e16 = dop != manta::OP_DOT ? 1 : 0;
    if (plan.use) {
        int rc = run_mq(rt, c, dop, order, q, nq, k, plan, nullptr, out_ids, out_scores, err, any_order && !out_acc);
        if (rc) return rc;
        if (out_acc)
            LAUNCH_TRY(manta::launch_q8_rescore((const int8_t*)c->codes, c->pitch, 0, c->n, (int)c->d, q, out_ids,
                                                (int)k, (int)nq, e16, out_acc, rt->stream),
                       "q8_rescore");
        return MANTA_ROCM_OK;
    }
    StreamTopk st = stream_topk_shape(c, nq, k, choose_rounds((c->n + 255) / 256, nq, rt->cus));
    uint64_t* partial = nullptr;
    int rc = take_buffer(rt, sc, (size_t)nq * st.parts * k * 8, (void**)&partial, err);
    if (rc) return rc;
    ScanArgs a = stream_topk_args(c, q, st, k, order, out_ids, out_scores, partial, sc ? sc->tickets : rt->tickets);
    // small k on the coalesced q8 kernel: sorted per-wave lists in registers
    // (LDS only for merging the waves' lists)
    if (c->format == MANTA_ROCM_Q8_ROWS && manta::q8_scan_coalesced(c->pitch) && k <= manta::kWaveListMaxK) {
        a.wave_lists = 1;
        a.lds_keys = 256;
    }
    rc = launch_scan(rt, c, dop, a, dim3((unsigned)st.parts, (unsigned)nq), (size_t)a.lds_keys * 8, err);
    if (rc) return rc;
    if (out_acc) {
        LAUNCH_TRY(manta::launch_q8_rescore((const int8_t*)c->codes, c->pitch, c->sets == 1 ? 0 : c->n, c->n,
                                            (int)c->d, q, out_ids, (int)k, (int)nq, e16, out_acc, rt->stream),
                   "q8_rescore");
    }
    return MANTA_ROCM_OK;
}

// Reference-semantics top-k.  The quantized-query scan returns its best kp
// rows; ref_finish rescores them with the reference arithmetic and proves
// (or not) that they hold the reference's best k; queries it cannot prove
// are rescanned in full with the reference arithmetic.  Candidates whose
// scales lie outside the range the scan's error bounds assume skip the scan
// and are rescanned in full.
int ref_topk(MantaRocm* rt, const MantaRocmCandidates* c, const ScoreOp& so, int order, const uint16_t* q,
             int64_t nq, int64_t k, int32_t* out_ids, float* out_scores, manta_rt::Scratch* sc, char** err) {
    const int fmt = c->format == MANTA_ROCM_Q8_ROWS ? 8 : 4;
    const int smallest = order == MANTA_ROCM_SMALLEST;
    int* redo = nullptr;
    uint64_t* redo_tau = nullptr;
    if (c->ref_ranked) {
        // a margin of rows past the k-th: ties and near-ties of the scan
        // scores across the kp-th row are what would send a query to the
        // full rescan.  A margin that would just pass a power of two stops
        // there (at least 8 rows): the finish sorts next_pow2(kp) keys, and
        // 1024 of them take one per thread where 1031 would take two.
        int64_t margin = k + std::max<int64_t>(8, k / 32);
        int64_t p2 = 1;
        while (p2 < k) p2 <<= 1;
        if (p2 >= k + 8 && p2 < margin) margin = p2;
        const int64_t kp = std::min<int64_t>(std::min<int64_t>(c->n, kMaxDeviceK), margin);
        const size_t need = (size_t)nq * kp * 16 + (size_t)nq * 12 + 2048;
        char* base = nullptr;
        int rc = sc ? take_buffer(rt, sc, need, (void**)&base, err) : ensure_ref_workspace(rt, need, err);
        if (rc) return rc;
        Carver cv(sc ? (void*)base : rt->ws_ref);
        int32_t* cand_ids = cv.take<int32_t>((size_t)nq * kp);
        float* cand_scores = cv.take<float>((size_t)nq * kp);
        uint64_t* cand_keys = cv.take<uint64_t>((size_t)nq * kp);
        redo = cv.take<int>((size_t)nq);
        redo_tau = cv.take<uint64_t>((size_t)nq);
        // (in any order: ref_finish sorts the rescored keys and reads only the
        // kp-th, worst, scan score)
        rc = scan_topk(rt, c, so.scan, order, q, nq, kp, cand_ids, cand_scores, nullptr, sc, err, true);
        if (rc) return rc;
        manta::RefArgs ra{};
        ra.fmt = fmt;
        ra.codes = c->codes;
        ra.scales = c->scales;
        ra.sqd = c->sqd;
        ra.n = c->n;
        ra.pitch = c->pitch;
        ra.d = (int)c->d;
        ra.set_stride = c->sets == 1 ? 0 : c->n;
        ra.queries = q;
        ra.nq = (int)nq;
        ra.op = so.ref;
        ra.smallest = smallest;
        ra.k = (int)k;
        ra.kp = (int)kp;
        ra.cand_ids = cand_ids;
        ra.cand_scores = cand_scores;
        // relative error of the scan's q^.d' term: q8 three f32 roundings
        // (scale*qs, f32(acc), the product); q4 an fma per block plus the
        // final product
        ra.e_qd = fmt == 8 ? 3.1f * 0x1p-24f : ((float)c->nb + 1.2f) * 0x1p-24f;
        ra.maxdn = c->maxdn;
        ra.maxdd = c->maxdd;
        ra.out_ids = out_ids;
        ra.out_scores = out_scores;
        ra.redo = redo;
        ra.redo_tau = redo_tau;
        LAUNCH_TRY(manta::launch_ref_rescore(ra, cand_keys, rt->stream), "ref_rescore");
        LAUNCH_TRY(manta::launch_ref_finish(ra, cand_keys, rt->stream), "ref_finish");
    }
    // The full rescan of the queries the finish marked: parts of up to 64
    // rounds per query, and R query slots, each taking every R-th query, so
    // that about 256 workgroups check the marks when nothing is marked (all
    // queries when the scans were skipped).
    const int64_t tiles = (c->n + 255) / 256;
    const int rounds = (int)std::max<int64_t>(1, std::min<int64_t>(64, (tiles + 63) / 64));
    StreamTopk st = stream_topk_shape(c, nq, k, rounds);
    const int64_t R = redo ? std::max<int64_t>(1, std::min<int64_t>(nq, 256 / std::max<int64_t>(1, st.parts)))
                           : std::min<int64_t>(nq, 65535);
    uint64_t* partial = nullptr;
    int rc = take_buffer(rt, sc, (size_t)nq * st.parts * k * 8, (void**)&partial, err);
    if (rc) return rc;
    ScanArgs a = stream_topk_args(c, q, st, k, order, out_ids, out_scores, partial, sc ? sc->tickets : rt->tickets);
    LAUNCH_TRY(manta::launch_ref_scan(fmt, so.ref, a, (int)nq, c->sqd, redo, redo_tau,
                                      dim3((unsigned)st.parts, (unsigned)R), (size_t)a.lds_keys * 8, rt->stream),
               "ref_scan");
    return MANTA_ROCM_OK;
}

}  // namespace

extern "C" {

int manta_rocm_score_topk(MantaRocm* rt, const MantaRocmCandidates* c, int op, int order,
                          const uint16_t* q, int64_t nq, int64_t k, int32_t* out_ids,
                          float* out_scores, int64_t* out_acc, char** err) {
    return manta_rt::score_topk_impl(rt, c, op, order, q, nq, k, out_ids, out_scores, out_acc, nullptr, err);
}

}  // extern "C"

int manta_rt::score_topk_impl(MantaRocm* rt, const MantaRocmCandidates* c, int op, int order, const uint16_t* q,
                              int64_t nq, int64_t k, int32_t* out_ids, float* out_scores, int64_t* out_acc,
                              Scratch* sc, char** err) {
    RT_CHECK(rt);
    int rc = check_score_args(c, op, q, nq, err);
    if (rc) return rc;
    if (order != MANTA_ROCM_LARGEST && order != MANTA_ROCM_SMALLEST)
        return fail(err, MANTA_ROCM_ERROR, "unknown topk order %d", order);
    if (k <= 0 || k > c->n)
        return fail(err, MANTA_ROCM_ERROR, "topk limit %lld out of range for row width %lld",
                    (long long)k, (long long)c->n);
    if (k > kMaxDeviceK)
        return fail(err, MANTA_ROCM_UNSUPPORTED, "topk limit %lld exceeds the device maximum %lld",
                    (long long)k, (long long)kMaxDeviceK);
    if (!out_ids) return fail(err, MANTA_ROCM_ERROR, "nil topk output");
    const ScoreOp so = parse_op(c, op);
    if (out_acc && (c->format != MANTA_ROCM_Q8_ROWS || !so.quant))
        return fail(err, MANTA_ROCM_ERROR, "accumulator output needs q8 candidates and quantized-query scores");
    if (!sc) {
        if (so.quant) return scan_topk(rt, c, so.scan, order, q, nq, k, out_ids, out_scores, out_acc, nullptr, err);
        return ref_topk(rt, c, so, order, q, nq, k, out_ids, out_scores, nullptr, err);
    }
    // the allocation-free path: no per-launch timing events either
    const bool timing = rt->timing;
    rt->timing = false;
    rc = so.quant ? scan_topk(rt, c, so.scan, order, q, nq, k, out_ids, out_scores, out_acc, sc, err)
                  : ref_topk(rt, c, so, order, q, nq, k, out_ids, out_scores, sc, err);
    rt->timing = timing;
    return rc;
}

int manta_rt::runtime_device(const MantaRocm* rt) { return rt ? rt->device : -1; }

void* manta_rt::runtime_stream(const MantaRocm* rt) { return rt ? (void*)rt->stream : nullptr; }

int manta_rt::pack_candidates_into(MantaRocm* rt, const MantaRocmCandidates* c, const int32_t* top, int64_t nq,
                                   int64_t k, const int64_t* candidate_ids, int64_t* out_ids, void* out_rows,
                                   void* out_scales, unsigned long long* err_word, char** err) {
    RT_CHECK(rt);
    if (!c || !top || !out_rows || !out_scales) return fail(err, MANTA_ROCM_ERROR, "nil pack_candidates input");
    if (nq <= 0 || k <= 0) return fail(err, MANTA_ROCM_ERROR, "pack_candidates expects nq > 0 and k > 0");
    if (c->sets != 1 && c->sets != nq)
        return fail(err, MANTA_ROCM_ERROR, "pack_candidates: %lld queries for %lld candidate sets", (long long)nq,
                    (long long)c->sets);
    if (out_ids && !candidate_ids) return fail(err, MANTA_ROCM_ERROR, "pack_candidates: ids output without candidate ids");
    manta::PackArgs a{};
    a.top = top;
    a.nq = nq;
    a.k = k;
    a.n = c->n;
    a.sets = (int)c->sets;
    a.codes = (const uint8_t*)c->codes;
    a.pitch = c->pitch;
    a.row_bytes = c->format == MANTA_ROCM_Q8_ROWS ? (int)c->d : (int)(c->d / 2);
    a.scales = (const uint8_t*)c->scales;
    a.scale_bytes = c->format == MANTA_ROCM_Q8_ROWS ? 4 : (int)(c->nb * 2);
    a.ids = candidate_ids;
    a.ids_out = out_ids;
    a.rows_out = (uint8_t*)out_rows;
    a.scales_out = (uint8_t*)out_scales;
    a.err = err_word;
    LAUNCH_TRY(manta::launch_pack_candidates(a, rt->stream), "pack_candidates");
    return MANTA_ROCM_OK;
}

extern "C" {

int manta_rocm_pack_candidates(MantaRocm* rt, const MantaRocmCandidates* c, const int32_t* top, int64_t nq,
                               int64_t k, const int64_t* candidate_ids, int64_t* out_ids, void* out_rows,
                               void* out_scales, char** err) {
    RT_CHECK(rt);
    const int rc = manta_rt::pack_candidates_into(rt, c, top, nq, k, candidate_ids, out_ids, out_rows, out_scales,
                                                  rt->err_word, err);
    if (rc == MANTA_ROCM_OK) rt->gather_pending = true;
    return rc;
}

int manta_rocm_topk(MantaRocm* rt, const float* scores, int64_t rows, int64_t cols, int64_t k,
                    int order, int32_t* out_ids, float* out_values, char** err) {
    RT_CHECK(rt);
    if (!scores) return fail(err, MANTA_ROCM_ERROR, "nil topk input");
    if (rows <= 0 || cols <= 0) return fail(err, MANTA_ROCM_ERROR, "topk expects rank-1 or rank-2 scores");
    if (order != MANTA_ROCM_LARGEST && order != MANTA_ROCM_SMALLEST)
        return fail(err, MANTA_ROCM_ERROR, "unknown topk order %d", order);
    if (k <= 0 || k > cols) {
        if (rows == 1)
            return fail(err, MANTA_ROCM_ERROR, "topk limit %lld out of range for %lld scores",
                        (long long)k, (long long)cols);
        return fail(err, MANTA_ROCM_ERROR, "topk limit %lld out of range for row width %lld",
                    (long long)k, (long long)cols);
    }
    if (k > kMaxDeviceK)
        return fail(err, MANTA_ROCM_UNSUPPORTED, "topk limit %lld exceeds the device maximum %lld",
                    (long long)k, (long long)kMaxDeviceK);
    if (rows > 65535) return fail(err, MANTA_ROCM_UNSUPPORTED, "more than 65535 score rows");
    if (!out_ids) return fail(err, MANTA_ROCM_ERROR, "nil topk output");
    const int64_t tiles = (cols + 255) / 256;
    int64_t want_parts = std::max<int64_t>(1, 1024 / rows);
    int64_t rounds = std::max<int64_t>(1, (tiles + want_parts - 1) / want_parts);
    rounds = std::min<int64_t>(rounds, std::max<int64_t>(1, tiles));
    const int64_t seg = rounds * 256;
    const int64_t parts = (cols + seg - 1) / seg;
    const int cap = cap_for_k(k);
    int rc = ensure_workspace(rt, (size_t)rows * parts * k * 8 + 256, err);
    if (rc) return rc;
    uint64_t* partial = (uint64_t*)rt->ws;
    const int smallest = order == MANTA_ROCM_SMALLEST;
    LAUNCH_TRY(manta::launch_topk_rows_partial(scores, rows, cols, seg, (int)parts, (int)k, cap,
                                               smallest, partial, rt->stream),
               "topk_partial");
    LAUNCH_TRY(manta::launch_topk_merge(partial, rows, parts * k, (int)k, cap, smallest, out_ids,
                                        out_values, rt->stream),
               "topk_merge");
    return MANTA_ROCM_OK;
}

// ------------------------------------------------------ dense retrieval

namespace {

int check_dense(const void* rows, int dtype, int64_t n, int64_t d, const float* q, int64_t nq, int64_t qd,
                char** err) {
    if (!rows || !q) return fail(err, MANTA_ROCM_ERROR, "nil dense retrieval input");
    if (dtype != MANTA_ROCM_DENSE_F32 && dtype != MANTA_ROCM_DENSE_F16)
        return fail(err, MANTA_ROCM_ERROR, "unknown dense vector dtype %d", dtype);
    if (n <= 0 || d < 0 || nq <= 0 || qd < 0)
        return fail(err, MANTA_ROCM_ERROR, "dense retrieval: bad shape [%lld,%lld] x [%lld,%lld]", (long long)nq,
                    (long long)qd, (long long)n, (long long)d);
    if (std::min(d, qd) > 0x7FFFFFFF || n > ((int64_t)1 << 31) - 1)
        return fail(err, MANTA_ROCM_UNSUPPORTED, "dense retrieval: shape beyond the device path");
    return MANTA_ROCM_OK;
}

// Queries per score-matrix launch: the matrix stays within 512 MiB (and the
// grid's y extent within its limit).
int64_t dense_chunk(int64_t n, int64_t nq) {
    const int64_t by_bytes = std::max<int64_t>(1, ((int64_t)512 << 20) / (n * 4));
    return std::min<int64_t>(std::min<int64_t>(nq, by_bytes), (int64_t)65535 * 8);
}

}  // namespace

int manta_rocm_dense_scores(MantaRocm* rt, const void* rows, int dtype, int64_t n, int64_t d, const float* q,
                            int64_t nq, int64_t qd, float* out, char** err) {
    RT_CHECK(rt);
    int rc = check_dense(rows, dtype, n, d, q, nq, qd, err);
    if (rc) return rc;
    if (!out) return fail(err, MANTA_ROCM_ERROR, "nil dense retrieval output");
    const int len = (int)std::min(d, qd);
    const int64_t chunk = std::min<int64_t>(nq, (int64_t)65535 * 8);
    for (int64_t q0 = 0; q0 < nq; q0 += chunk) {
        const int nc = (int)std::min(chunk, nq - q0);
        LAUNCH_TRY(manta::launch_dense_dot(rows, dtype == MANTA_ROCM_DENSE_F16, n, d, len, q + q0 * qd, qd, nc,
                                           out + q0 * n, rt->stream),
                   "dense_dot");
    }
    return MANTA_ROCM_OK;
}

int manta_rocm_dense_topk(MantaRocm* rt, const void* rows, int dtype, int64_t n, int64_t d, const float* q,
                          int64_t nq, int64_t qd, int64_t k, int32_t* out_ids, float* out_scores, char** err) {
    RT_CHECK(rt);
    int rc = check_dense(rows, dtype, n, d, q, nq, qd, err);
    if (rc) return rc;
    if (!out_ids) return fail(err, MANTA_ROCM_ERROR, "nil topk output");
    if (k <= 0 || k > n) {
        if (nq == 1)
            return fail(err, MANTA_ROCM_ERROR, "topk limit %lld out of range for %lld scores", (long long)k,
                        (long long)n);
        return fail(err, MANTA_ROCM_ERROR, "topk limit %lld out of range for row width %lld", (long long)k,
                    (long long)n);
    }
    if (k > kMaxDeviceK)
        return fail(err, MANTA_ROCM_UNSUPPORTED, "topk limit %lld exceeds the device maximum %lld", (long long)k,
                    (long long)kMaxDeviceK);
    const int64_t chunk = std::min<int64_t>(dense_chunk(n, nq), 65535);
    rc = ensure_ref_workspace(rt, (size_t)(chunk * n) * 4 + 256, err);
    if (rc) return rc;
    float* scores = (float*)rt->ws_ref;
    for (int64_t q0 = 0; q0 < nq; q0 += chunk) {
        const int64_t nc = std::min(chunk, nq - q0);
        rc = manta_rocm_dense_scores(rt, rows, dtype, n, d, q + q0 * qd, nc, qd, scores, err);
        if (rc) return rc;
        rc = manta_rocm_topk(rt, scores, nc, n, k, MANTA_ROCM_LARGEST, out_ids + q0 * k,
                             out_scores ? out_scores + q0 * k : nullptr, err);
        if (rc) return rc;
    }
    return MANTA_ROCM_OK;
}

// ---------------------------------------------------------------- embed

namespace {

bool proj_q8(int kind) { return kind == MANTA_ROCM_PROJ_Q8_COL || kind == MANTA_ROCM_PROJ_Q8_COL_T; }
bool proj_prepared(int kind) { return kind == MANTA_ROCM_PROJ_F16_T || kind == MANTA_ROCM_PROJ_Q8_COL_T; }

int check_proj(int proj_kind, const void* proj, const float* col_scale, int64_t k, int64_t n, char** err) {
    if (!proj) return fail(err, MANTA_ROCM_ERROR, "nil matmul input");
    if (proj_kind < MANTA_ROCM_PROJ_F16 || proj_kind > MANTA_ROCM_PROJ_Q8_COL_T)
        return fail(err, MANTA_ROCM_ERROR, "unknown projection kind %d", proj_kind);
    if (proj_q8(proj_kind) && !col_scale)
        return fail(err, MANTA_ROCM_ERROR, "q8 projection needs per-column scales");
    if (k <= 0 || n <= 0) return fail(err, MANTA_ROCM_ERROR, "matmul mismatch: empty operand");
    if (k % 8 != 0)
        return fail(err, MANTA_ROCM_UNSUPPORTED, "matmul: inner dimension %lld is not a multiple of 8",
                    (long long)k);
    if (n % (proj_q8(proj_kind) ? 4 : 2) != 0)
        return fail(err, MANTA_ROCM_UNSUPPORTED, "matmul: output width %lld not supported", (long long)n);
    if (n > 4096 || k > (1 << 20))
        return fail(err, MANTA_ROCM_UNSUPPORTED, "matmul: shape beyond the device path");
    return MANTA_ROCM_OK;
}

}  // namespace

int manta_rocm_gather_rows_f16(MantaRocm* rt, const uint16_t* table, int64_t vocab, int64_t d,
                               const int32_t* idx, int64_t nidx, uint16_t* out, char** err) {
    RT_CHECK(rt);
    if (!table || !idx || !out) return fail(err, MANTA_ROCM_ERROR, "nil gather input");
    if (vocab <= 0 || d <= 0 || nidx <= 0)
        return fail(err, MANTA_ROCM_ERROR, "gather expects i32 indices");
    if (nidx > 0x7FFFFFFF) return fail(err, MANTA_ROCM_UNSUPPORTED, "gather: too many indices");
    LAUNCH_TRY(manta::launch_gather_rows_f16(table, vocab, d, idx, nidx, out, rt->err_word, rt->stream),
               "gather");
    rt->gather_pending = true;
    return MANTA_ROCM_OK;
}

int manta_rocm_matmul_f16(MantaRocm* rt, const uint16_t* lhs, int64_t m, int64_t k, const void* rhs,
                          int proj_kind, const float* col_scale, int64_t n, float* out, char** err) {
    RT_CHECK(rt);
    if (!lhs || !out) return fail(err, MANTA_ROCM_ERROR, "nil matmul input");
    if (m <= 0) return fail(err, MANTA_ROCM_ERROR, "matmul mismatch: empty operand");
    int rc = check_proj(proj_kind, rhs, col_scale, k, n, err);
    if (rc) return rc;
    if ((m + 63) / 64 > 0x7FFFFFFF) return fail(err, MANTA_ROCM_UNSUPPORTED, "matmul: too many rows");
    manta::EmbedArgs a{};
    a.A = lhs;
    a.M = m;
    a.K = (int)k;
    a.N = (int)n;
    a.B = rhs;
    a.colscale = col_scale;
    a.Y = out;
    const bool q8b = proj_q8(proj_kind);
    if (proj_prepared(proj_kind)) {
        // the operand is already f16 [n][k]: the pipelined GEMM only
        if (!manta::embed_gemm2_supported(a))
            return fail(err, MANTA_ROCM_UNSUPPORTED,
                        "matmul: a prepared projection needs k %% 32 == 0 and n %% 128 == 0 (got %lld x %lld)",
                        (long long)k, (long long)n);
        LAUNCH_TRY(manta::launch_embed_gemm2(a, false, q8b, false, (const uint16_t*)rhs, rt->stream), "matmul");
        return MANTA_ROCM_OK;
    }
    if (manta::embed_gemm3_supported(a, q8b)) {
        LAUNCH_TRY(manta::launch_embed_gemm3(a, false, false, rt->stream), "matmul");
        return MANTA_ROCM_OK;
    }
    if (manta::embed_gemm2_supported(a)) {
        rc = ensure_workspace(rt, (size_t)n * k * 2 + 256, err);
        if (rc) return rc;
        LAUNCH_TRY(manta::launch_embed_transpose_b(a, q8b, (uint16_t*)rt->ws, rt->stream), "embed_transpose");
        LAUNCH_TRY(manta::launch_embed_gemm2(a, false, q8b, false, (const uint16_t*)rt->ws, rt->stream), "matmul");
        return MANTA_ROCM_OK;
    }
    LAUNCH_TRY(manta::launch_embed_gemm(a, false, q8b, false, rt->stream), "matmul");
    return MANTA_ROCM_OK;
}

int manta_rocm_mean_pool_masked(MantaRocm* rt, const float* x, const int32_t* mask, int64_t b,
                                int64_t t, int64_t c, float* out, char** err) {
    RT_CHECK(rt);
    if (!x) return fail(err, MANTA_ROCM_ERROR, "nil mean_pool input");
    if (!mask) return fail(err, MANTA_ROCM_ERROR, "nil mean_pool mask");
    if (!out) return fail(err, MANTA_ROCM_ERROR, "nil mean_pool output");
    if (b <= 0 || t <= 0 || c <= 0) return fail(err, MANTA_ROCM_ERROR, "mean_pool expects rank-2 or rank-3 tensor input");
    LAUNCH_TRY(manta::launch_mean_pool_masked(x, mask, b, t, c, out, rt->stream), "mean_pool");
    return MANTA_ROCM_OK;
}

int manta_rocm_mean_pool(MantaRocm* rt, const float* x, int64_t b, int64_t t, int64_t c, float* out, char** err) {
    RT_CHECK(rt);
    if (!x) return fail(err, MANTA_ROCM_ERROR, "nil mean_pool input");
    if (!out) return fail(err, MANTA_ROCM_ERROR, "nil mean_pool output");
    if (b <= 0 || t <= 0 || c <= 0) return fail(err, MANTA_ROCM_ERROR, "mean_pool expects rank-2 or rank-3 tensor input");
    LAUNCH_TRY(manta::launch_mean_pool(x, b, t, c, out, rt->stream), "mean_pool");
    return MANTA_ROCM_OK;
}

int manta_rocm_normalize_rows(MantaRocm* rt, float* x, int64_t rows, int64_t cols, char** err) {
    RT_CHECK(rt);
    if (!x) return fail(err, MANTA_ROCM_ERROR, "nil normalize input");
    if (rows <= 0 || cols <= 0) return MANTA_ROCM_OK;
    LAUNCH_TRY(manta::launch_normalize_rows(x, rows, cols, rt->stream), "normalize");
    return MANTA_ROCM_OK;
}

int manta_rocm_encoder_pooled(MantaRocm* rt, const int32_t* tokens, const int32_t* mask, int64_t b, int64_t t,
                              const MantaRocmEncoderWeights* w, int64_t vocab, int64_t d, int64_t h,
                              uint16_t* out, char** err) {
    return manta_rocm_encoder_pooled_layers(rt, tokens, mask, b, t, w, vocab, d, h, 1, out, err);
}

int manta_rocm_encoder_pooled_layers(MantaRocm* rt, const int32_t* tokens, const int32_t* mask, int64_t b,
                                     int64_t t, const MantaRocmEncoderWeights* w, int64_t vocab, int64_t d,
                                     int64_t h, int64_t layers, uint16_t* out, char** err) {
    RT_CHECK(rt);
    if (layers < 1 || layers > 64) return fail(err, MANTA_ROCM_ERROR, "encoder: %lld layers", (long long)layers);
    if (!tokens || !mask || !w || !out) return fail(err, MANTA_ROCM_ERROR, "nil encoder input");
    if (!w->token_codes || !w->token_scales) return fail(err, MANTA_ROCM_ERROR, "nil encoder token table");
    for (int i = 0; i < 6; i++)
        if (!w->codes[i] || !w->col_scales[i]) return fail(err, MANTA_ROCM_ERROR, "nil encoder weight %d", i);
    if (b <= 0 || t <= 0 || vocab <= 0 || d <= 0 || h <= 0)
        return fail(err, MANTA_ROCM_ERROR, "encoder: bad shape b=%lld t=%lld vocab=%lld d=%lld h=%lld",
                    (long long)b, (long long)t, (long long)vocab, (long long)d, (long long)h);
    const int64_t rows = b * t;
    // the GEMM grids: 64-row tiles of the b*t rows (and of each sequence's t
    // rows for the attention products) in at most 65535 workgroup rows
    if (b > 65535 || rows > 0x7FFFFFFF || d > 0x7FFFFFFF || h > 0x7FFFFFFF || t > 0x7FFFFFFF ||
        (rows + 63) / 64 > 65535)
        return fail(err, MANTA_ROCM_UNSUPPORTED, "encoder: shape too large");
    // The weight GEMMs run on the f16 matrix cores when d and h are multiples
    // of 128 (embed_gemm2: the q8 weights widened exactly to f16 [N][K],
    // their column scales applied after the f32 accumulation; the left
    // operands rounded to f16 by the steps that produce them), else on the
    // f32 matrix cores (enc_gemm_mfma_kernel).  The attention products stay
    // f32.
    const bool f16w = d % 128 == 0 && h % 128 == 0 && d <= 4096 && h <= 8192;
    // x, q, k, v, mixed [rows, d]; scores [b, t, t]; ffn [rows, h]; pooled [b, d]
    // (f16 path: x16, k16, mx16 [rows, d], ffn16 [rows, h], the six weights as f16 [N][K])
    const size_t rd = (size_t)rows * (size_t)d;
    const size_t wsz[6] = {(size_t)d * d, (size_t)d * d, (size_t)d * d, (size_t)d * d, (size_t)d * h, (size_t)h * d};
    const size_t ffn_f32 = f16w ? 1 : (size_t)rows * h;  // the f16 path keeps ffn in f16 only
    size_t need = 5 * (rd * 4 + 256) + (size_t)b * t * t * 4 + 256 + ffn_f32 * 4 + 256 + (size_t)b * d * 4 + 256;
    if (f16w) {
        need += 3 * (rd * 2 + 256) + (size_t)rows * h * 2 + 256;
        for (size_t z : wsz) need += z * 2 + 256;
    }
    int rc = ensure_workspace(rt, need, err);
    if (rc) return rc;
    Carver cv(rt->ws);
    float* x = cv.take<float>(rd);
    float* q = cv.take<float>(rd);
    float* k = cv.take<float>(rd);
    float* v = cv.take<float>(rd);
    float* mx = cv.take<float>(rd);
    float* sc = cv.take<float>((size_t)b * t * t);
    float* ffn = cv.take<float>(ffn_f32);
    float* pooled = cv.take<float>((size_t)b * d);
    uint16_t *x16 = nullptr, *k16 = nullptr, *mx16 = nullptr, *ffn16 = nullptr, *wt[6] = {};
    if (f16w) {
        x16 = cv.take<uint16_t>(rd);
        k16 = cv.take<uint16_t>(rd);
        mx16 = cv.take<uint16_t>(rd);
        ffn16 = cv.take<uint16_t>((size_t)rows * h);
        for (int i = 0; i < 6; i++) wt[i] = cv.take<uint16_t>(wsz[i]);
    }
    const int R = (int)rows, D = (int)d, H = (int)h, T = (int)t;
    const int64_t td = (int64_t)t * d, tt = (int64_t)t * t;
    hipStream_t s = rt->stream;
    // out = in16 [R, K] x weight i (f16 [N][K], column scales) on f16 MFMA:
    // f32 out, or f16 out with gelu applied (ffn_up)
    auto wgemm = [&](int i, const uint16_t* in16, int K, int N, float* out, uint16_t* out16, bool gelu) {
        manta::EmbedArgs ea{};
        ea.A = in16;
        ea.M = R;
        ea.K = K;
        ea.N = N;
        ea.colscale = w->col_scales[i];
        ea.Y = out;
        ea.Y16 = out16;
        ea.gelu = gelu ? 1 : 0;
        return manta::launch_embed_gemm2(ea, false, true, false, wt[i], s);
    };
    if (f16w) {
        const int kn[6][2] = {{D, D}, {D, D}, {D, D}, {D, D}, {D, H}, {H, D}};
        for (int i = 0; i < 6; i++) {
            manta::EmbedArgs ea{};
            ea.K = kn[i][0];
            ea.N = kn[i][1];
            ea.B = w->codes[i];
            LAUNCH_TRY(manta::launch_embed_transpose_b(ea, true, wt[i], s), "embed_transpose");
        }
    }
    LAUNCH_TRY(manta::launch_enc_gather_q8(tokens, rows, w->token_codes, w->token_scales, vocab, D, x, rt->err_word, s,
                                           x16),
               "encoder_gather");
    rt->gather_pending = true;
    for (int64_t layer = 0; layer < layers; layer++) {
    if (layer > 0) std::swap(x, mx);  // this block's hidden input is the last block's encoded output
    if (f16w) {
        LAUNCH_TRY(wgemm(0, x16, D, D, q, nullptr, false), "encoder_gemm");
        LAUNCH_TRY(wgemm(1, x16, D, D, k, nullptr, false), "encoder_gemm");
        LAUNCH_TRY(wgemm(2, x16, D, D, v, nullptr, false), "encoder_gemm");
    } else {
        LAUNCH_TRY(manta::launch_enc_gemm(1, x, 0, w->codes[0], w->col_scales[0], 0, q, 0, R, D, D, 1, s), "encoder_gemm");
        LAUNCH_TRY(manta::launch_enc_gemm(1, x, 0, w->codes[1], w->col_scales[1], 0, k, 0, R, D, D, 1, s), "encoder_gemm");
        LAUNCH_TRY(manta::launch_enc_gemm(1, x, 0, w->codes[2], w->col_scales[2], 0, v, 0, R, D, D, 1, s), "encoder_gemm");
    }
    // scores[b] = q[b] @ transpose(k[b]); softmax over each row of t
    LAUNCH_TRY(manta::launch_enc_gemm(2, q, td, k, nullptr, td, sc, tt, T, T, D, (int)b, s), "encoder_attention");
    LAUNCH_TRY(manta::launch_enc_softmax_rows(sc, rows, T, s), "encoder_softmax");
    LAUNCH_TRY(manta::launch_enc_gemm(0, sc, tt, v, nullptr, td, mx, td, T, D, T, (int)b, s, false, mx16),
               "encoder_attention");
    // attended = mixed @ attn_o (into q); attn_hidden = layernorm(attended + x) (into k)
    if (f16w) LAUNCH_TRY(wgemm(3, mx16, D, D, q, nullptr, false), "encoder_gemm");
    else LAUNCH_TRY(manta::launch_enc_gemm(1, mx, 0, w->codes[3], w->col_scales[3], 0, q, 0, R, D, D, 1, s), "encoder_gemm");
    LAUNCH_TRY(manta::launch_enc_add_layernorm(q, x, k, rows, D, s, k16), "encoder_layernorm");
    // projected = gelu @ projection (into v); encoded = layernorm(projected + attn_hidden) (into mx, and its
    // f16 copy into x16, the next block's input)
    if (f16w) {
        LAUNCH_TRY(wgemm(4, k16, D, H, nullptr, ffn16, true), "encoder_gemm");
        LAUNCH_TRY(wgemm(5, ffn16, H, D, v, nullptr, false), "encoder_gemm");
    } else {
        LAUNCH_TRY(manta::launch_enc_gemm(1, k, 0, w->codes[4], w->col_scales[4], 0, ffn, 0, R, H, D, 1, s, true),
                   "encoder_gemm");
        LAUNCH_TRY(manta::launch_enc_gemm(1, ffn, 0, w->codes[5], w->col_scales[5], 0, v, 0, R, D, H, 1, s),
                   "encoder_gemm");
    }
    LAUNCH_TRY(manta::launch_enc_add_layernorm(v, k, mx, rows, D, s, x16), "encoder_layernorm");
    }
    LAUNCH_TRY(manta::launch_normalize_rows(mx, rows, d, s), "normalize");
    LAUNCH_TRY(manta::launch_mean_pool_masked(mx, mask, b, t, d, pooled, s), "mean_pool");
    LAUNCH_TRY(manta::launch_enc_to_f16(pooled, b * d, out, s), "encoder_out");
    return MANTA_ROCM_OK;
}

int manta_rocm_prepare_projection(MantaRocm* rt, const void* proj, int proj_kind, int64_t d, int64_t e,
                                  uint16_t* out, int* out_kind, char** err) {
    RT_CHECK(rt);
    if (!out || !out_kind) return fail(err, MANTA_ROCM_ERROR, "nil prepare_projection output");
    if (proj_kind != MANTA_ROCM_PROJ_F16 && proj_kind != MANTA_ROCM_PROJ_Q8_COL)
        return fail(err, MANTA_ROCM_ERROR, "prepare_projection: kind %d is not a [d, e] projection", proj_kind);
    // (the scales stay with the caller; check_proj only needs a non-null one)
    static const float kOne = 1.0f;
    int rc = check_proj(proj_kind, proj, &kOne, d, e, err);
    if (rc) return rc;
    manta::EmbedArgs a{};
    a.K = (int)d;
    a.N = (int)e;
    a.B = proj;
    LAUNCH_TRY(manta::launch_embed_transpose_b(a, proj_kind == MANTA_ROCM_PROJ_Q8_COL, out, rt->stream),
               "embed_transpose");
    *out_kind = proj_kind == MANTA_ROCM_PROJ_Q8_COL ? MANTA_ROCM_PROJ_Q8_COL_T : MANTA_ROCM_PROJ_F16_T;
    return MANTA_ROCM_OK;
}

int manta_rocm_embed_pooled(MantaRocm* rt, const int32_t* tokens, const int32_t* mask, int64_t b,
                            int64_t t, const uint16_t* table, int64_t vocab, int64_t d, const void* proj,
                            int proj_kind, const float* col_scale, int64_t e, uint16_t* out, char** err) {
    RT_CHECK(rt);
    if (!tokens || !table || !out) return fail(err, MANTA_ROCM_ERROR, "nil embed input");
    if (b <= 0 || t <= 0 || vocab <= 0)
        return fail(err, MANTA_ROCM_ERROR, "embed: bad shape [%lld,%lld] x [%lld,%lld]", (long long)b,
                    (long long)t, (long long)vocab, (long long)d);
    int rc = check_proj(proj_kind, proj, col_scale, d, e, err);
    if (rc) return rc;
    const bool q8b = proj_q8(proj_kind);
    const bool prepared = proj_prepared(proj_kind);
    manta::EmbedArgs a{};
    a.tokens = tokens;
    a.mask = mask;
    a.table = table;
    a.vocab = vocab;
    a.T = t;
    a.batches = b;
    a.K = (int)d;
    a.N = (int)e;
    a.B = proj;
    a.colscale = col_scale;
    a.err = rt->err_word;
    if (manta::embed_gemm5_supported(a) && b * t / 256 >= 128) {
        // many short sequences: 256-row workgroups of whole sequences finish
        // their embeddings themselves (after the projection's transpose,
        // unless it came prepared)
        a.out = out;
        const uint16_t* bt = (const uint16_t*)proj;
        if (!prepared) {
            rc = ensure_workspace(rt, (size_t)d * e * 2 + 256, err);
            if (rc) return rc;
            bt = (uint16_t*)rt->ws;
            LAUNCH_TRY(manta::launch_embed_transpose_b(a, q8b, (uint16_t*)rt->ws, rt->stream), "embed_transpose");
        }
        LAUNCH_TRY(manta::launch_embed_gemm5(a, q8b, bt, rt->stream), "embed");
        rt->gather_pending = true;
        return MANTA_ROCM_OK;
    }
    if (!prepared && manta::embed_gemm3_supported(a, q8b) && b <= kTickets) {
        // one launch: 128-row x 96-column tiles, the last tile of each
        // sequence finishes it (every operand in one round of loads when K
        // allows, else a K ring)
        a.tiles_per_seq = (int)((t + 127) / 128);
        if (b * a.tiles_per_seq * 4 > 0x7FFFFFFF) return fail(err, MANTA_ROCM_UNSUPPORTED, "embed: batch too large");
        const bool one_round = manta::embed_gemm7_supported(a);
        rc = ensure_workspace(rt, align_up((size_t)(b * a.tiles_per_seq * (e + 1)) * sizeof(float), 256), err);
        if (rc) return rc;
        a.P = (float*)rt->ws;
        a.tickets = rt->tickets;
        a.out = out;
        if (one_round) LAUNCH_TRY(manta::launch_embed_gemm7(a, rt->stream), "embed");
        else LAUNCH_TRY(manta::launch_embed_gemm4(a, rt->stream), "embed");
        rt->gather_pending = true;
        return MANTA_ROCM_OK;
    }
    const int64_t tiles = (t + 63) / 64;
    if (b * tiles > 0x7FFFFFFF) return fail(err, MANTA_ROCM_UNSUPPORTED, "embed: batch too large");
    const size_t pbytes = align_up((size_t)(b * tiles * e) * sizeof(float), 256);
    rc = ensure_workspace(rt, pbytes + (size_t)d * e * 2 + 256, err);
    if (rc) return rc;
    a.tiles_per_seq = (int)tiles;
    a.P = (float*)rt->ws;
    if (prepared && !manta::embed_gemm2_supported(a))
        return fail(err, MANTA_ROCM_UNSUPPORTED,
                    "embed: a prepared projection needs d %% 32 == 0 and e %% 128 == 0 (got %lld x %lld)", (long long)d,
                    (long long)e);
    if (manta::embed_gemm2_supported(a)) {
        // the projection as f16 [e][d]: prepared, or transposed after the
        // partials
        const uint16_t* bt = (const uint16_t*)proj;
        if (!prepared) {
            uint16_t* w = (uint16_t*)((char*)rt->ws + pbytes);
            LAUNCH_TRY(manta::launch_embed_transpose_b(a, q8b, w, rt->stream), "embed_transpose");
            bt = w;
        }
        LAUNCH_TRY(manta::launch_embed_gemm2(a, true, q8b, true, bt, rt->stream), "embed");
    } else {
        LAUNCH_TRY(manta::launch_embed_gemm(a, true, q8b, true, rt->stream), "embed");
    }
    LAUNCH_TRY(manta::launch_embed_finalize(a.P, (int)tiles, mask, b, t, (int)e, out, rt->stream),
               "embed_finalize");
    rt->gather_pending = true;
    return MANTA_ROCM_OK;
}

}  // extern "C"
