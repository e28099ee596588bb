// noalloc.hip -- manta_rocm_score_topk_noalloc, the fused score + top-k that
// allocates nothing: for callers that cannot call hipMalloc (code under HIP
// graph capture, tight serving loops, harnesses that forbid allocation).
//
// Every scratch buffer of the call -- the streaming scans' per-workgroup
// keys, their last-workgroup tickets, and for reference scores the scan's
// candidates and the finish's verdicts -- is carved from `scratch`, a
// file-scope device array of kScratchBytes held by every GPU the library
// runs on until the process ends.  In host code the array's name is only a
// stand-in: its device address on each GPU is looked up once per device,
// with that device current, when a runtime is created (noalloc_init), and
// only that address is handed to kernels.  The array keeps the last call's
// contents; the kernels reset the tickets they use, and every other buffer
// is written before it is read within a call.  Calls that overlap on one GPU
// (two runtimes, or two streams) share the array and race.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <mutex>

#include "manta_rocm.h"
#include "runtime_internal.hpp"

namespace {

constexpr size_t kTicketBytes = (size_t)65536 * 4;  // one ticket per query
constexpr size_t kScratchBytes = (size_t)32 << 20;  // 32 MiB per GPU, tickets included

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};
hipError_t g_err[kMaxDevices] = {};
bool g_done[kMaxDevices] = {};

}  // namespace

// Look up this device's address of `scratch` (called by manta_rocm_create
// with `device` current; once per device).
void manta_rt::noalloc_init(int device) {
    if (device < 0 || device >= kMaxDevices) return;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_done[device]) return;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_ptr[device] = e == hipSuccess ? p : nullptr;
    g_err[device] = e;
    g_done[device] = true;
}

extern "C" int manta_rocm_score_topk_noalloc(MantaRocm* rt, const MantaRocmCandidates* cands, int op, int order,
                                             const uint16_t* queries_dev, int64_t nq, int64_t k,
                                             int32_t* out_ids_dev, float* out_scores_dev, int64_t* out_acc_dev,
                                             char** err) {
    const int device = manta_rt::runtime_device(rt);
    void* base = nullptr;
    hipError_t e = hipErrorInvalidDevice;
    if (device >= 0 && device < kMaxDevices) {
        std::lock_guard<std::mutex> lk(g_mu);
        if (g_done[device]) {
            base = g_ptr[device];
            e = g_err[device];
        }
    }
    if (!base) {
        if (err) {
            const char* why = rt ? hipGetErrorName(e) : "nil rocm runtime";
            const size_t n = 160;
            *err = (char*)malloc(n);
            if (*err) snprintf(*err, n, "score_topk_noalloc: allocation-free scratch unavailable on device %d (%s)",
                               device, why);
        }
        return MANTA_ROCM_ERROR;
    }
    manta_rt::Scratch sc;
    sc.tickets = (uint32_t*)base;
    sc.base = (char*)base + kTicketBytes;
    sc.bytes = kScratchBytes - kTicketBytes;
    return manta_rt::score_topk_impl(rt, cands, op, order, queries_dev, nq, k, out_ids_dev, out_scores_dev,
                                     out_acc_dev, &sc, err);
}

size_t manta_rt::noalloc_scratch_bytes() { return kScratchBytes - kTicketBytes; }
