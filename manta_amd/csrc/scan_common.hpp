// scan_common.hpp -- the end of a streaming top-k scan workgroup: publish
// its best keys and, in the last workgroup of a query, merge every part into
// the final ids (shared by kernels_score.hip and kernels_ref.hip).
#pragma once

#include "device_common.hpp"
#include "kernels.hpp"

namespace manta {

// Kernels that keep the encoded query in registers.
struct ScanTopkLds {
    TopKShared st;
    int last;
};

// End of a top-k scan workgroup: publish its k best keys; the last
// workgroup of the query (ticket == gridDim.x - 1) merges every part into
// the final sorted ids / scores and resets the ticket for the next call.
// Publication avoids device-wide fences (each one writes back and
// invalidates a whole XCD L2): the keys are stored write-through at agent
// scope (sc1), every thread waits for its stores to complete before the
// barrier, the ticket is an agent-scope atomic, and the merging workgroup
// reads the parts with agent-scope (sc1) loads.
template <class SL>
__device__ inline void finish_topk(const ScanArgs& a, uint64_t* keys, SL& S, int qi) {
    __syncthreads();
    topk_compact(keys, &S.st, a.k);
    const int64_t per_q = (int64_t)gridDim.x * a.k;
    uint64_t* dst = a.partial + (int64_t)qi * per_q + (int64_t)blockIdx.x * a.k;
    for (int i = threadIdx.x; i < a.k; i += blockDim.x)
        __hip_atomic_store(dst + i, i < S.st.cnt ? keys[i] : 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        S.last = __hip_atomic_fetch_add(&a.tickets[qi], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 gridDim.x - 1;
    __syncthreads();
    if (!S.last) return;
    const uint64_t* src = a.partial + (int64_t)qi * per_q;
    topk_init(keys, &S.st);
    if (per_q <= a.lds_keys) {
        // every part fits in LDS: one batch of loads, empty slots dropped
        for (int64_t base = 0; base < per_q; base += blockDim.x) {
            const int64_t i = base + threadIdx.x;
            const uint64_t key =
                i < per_q ? __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
            topk_offer(key, 0ull, keys, &S.st);
        }
        __syncthreads();
    } else {
        for (int64_t base = 0; base < per_q; base += blockDim.x) {
            const int64_t i = base + threadIdx.x;
            const uint64_t key =
                i < per_q ? __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
            topk_offer(key, S.st.tau, keys, &S.st);
            __syncthreads();
            topk_maybe_compact(keys, &S.st, a.k, a.cap);
        }
    }
    topk_compact(keys, &S.st, a.k);
    const int kept = S.st.cnt;
    topk_sort(keys, kept);
    for (int i = threadIdx.x; i < a.k; i += blockDim.x) {
        const uint64_t key = i < kept ? keys[i] : 0ull;
        a.out_ids[(int64_t)qi * a.k + i] = key ? (int32_t)key_index(key) : -1;
        if (a.out_topk_scores) a.out_topk_scores[(int64_t)qi * a.k + i] = key ? key_score(key, a.smallest) : 0.0f;
    }
    if (threadIdx.x == 0) __hip_atomic_store(&a.tickets[qi], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace manta
