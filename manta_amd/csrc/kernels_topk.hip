// kernels_topk.hip -- top-k selection (topKTensor, runtime/backend/
// tensor_ops.go:1523-1592) over f32 score rows, and the merge pass shared
// with the fused scoring kernels.
//
// Stage 1 (topk_rows_partial_kernel): grid (parts, rows); each workgroup
// streams a contiguous segment of one row in rounds of 256 scores through
// the LDS reservoir and emits its best k keys.  Stage 2 (topk_merge_kernel):
// one workgroup per row reduces parts*k keys to the final k, sorted by
// (value desc, index asc) -- or (value asc, index asc) for smallest-k -- and
// writes ids and values.  Keys make the order total, so the result does not
// depend on how rows were split across workgroups.
#include "device_common.hpp"
#include "kernels.hpp"

namespace manta {

__global__ __launch_bounds__(256) void topk_rows_partial_kernel(const float* __restrict__ scores,
                                                                int64_t cols, int64_t seg, int k,
                                                                int cap, int smallest,
                                                                uint64_t* __restrict__ partial) {
    extern __shared__ uint64_t keys[];
    __shared__ TopKShared st;
    const int64_t row = blockIdx.y;
    const float* src = scores + row * cols;
    const int64_t c0 = (int64_t)blockIdx.x * seg;
    int64_t c1 = c0 + seg;
    if (c1 > cols) c1 = cols;
    topk_init(keys, &st);
    for (int64_t base = c0; base < c1; base += blockDim.x) {
        const int64_t c = base + threadIdx.x;
        uint64_t key = 0;
        if (c < c1) key = make_key(src[c], (uint32_t)c, smallest);
        topk_offer(key, st.tau, keys, &st);
        __syncthreads();
        topk_maybe_compact(keys, &st, k, cap);
    }
    topk_compact(keys, &st, k);
    uint64_t* dst = partial + (row * gridDim.x + blockIdx.x) * k;
    for (int i = threadIdx.x; i < k; i += blockDim.x) dst[i] = i < st.cnt ? keys[i] : 0ull;
}

__global__ __launch_bounds__(256) void topk_merge_kernel(const uint64_t* __restrict__ partial,
                                                         int64_t per_row, int k, int cap,
                                                         int smallest, int32_t* __restrict__ ids,
                                                         float* __restrict__ values) {
    extern __shared__ uint64_t keys[];
    __shared__ TopKShared st;
    const int64_t row = blockIdx.x;
    const uint64_t* src = partial + row * per_row;
    topk_init(keys, &st);
    for (int64_t base = 0; base < per_row; base += blockDim.x) {
        const int64_t i = base + threadIdx.x;
        uint64_t key = i < per_row ? src[i] : 0ull;
        topk_offer(key, st.tau, keys, &st);
        __syncthreads();
        topk_maybe_compact(keys, &st, k, cap);
    }
    topk_compact(keys, &st, k);
    const int kept = st.cnt;
    topk_sort(keys, kept);
    for (int i = threadIdx.x; i < k; i += blockDim.x) {
        uint64_t key = i < kept ? keys[i] : 0ull;
        ids[row * k + i] = key ? (int32_t)key_index(key) : -1;
        if (values) values[row * k + i] = key ? key_score(key, smallest) : 0.0f;
    }
}

hipError_t launch_topk_rows_partial(const float* scores, int64_t rows, int64_t cols, int64_t seg,
                                    int parts, int k, int cap, int smallest, uint64_t* partial,
                                    hipStream_t s) {
    hipLaunchKernelGGL(topk_rows_partial_kernel, dim3(parts, (unsigned)rows), dim3(256),
                       (size_t)cap * sizeof(uint64_t), s, scores, cols, seg, k, cap, smallest,
                       partial);
    return hipGetLastError();
}

hipError_t launch_topk_merge(const uint64_t* partial, int64_t rows, int64_t per_row, int k, int cap,
                             int smallest, int32_t* ids, float* values, hipStream_t s) {
    hipLaunchKernelGGL(topk_merge_kernel, dim3((unsigned)rows), dim3(256),
                       (size_t)cap * sizeof(uint64_t), s, partial, per_row, k, cap, smallest, ids,
                       values);
    return hipGetLastError();
}

// ------------------------------------------------------ candidate pack

// One wave per (query, rank): the candidate id (int64), the packed row's
// bytes (4-byte words when row_bytes and pitch allow, else bytes) and its
// scales.  An index outside [0, n) zero-fills the slot and is reported.
__global__ __launch_bounds__(256) void pack_candidates_kernel(PackArgs a) {
    const int64_t slot = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (slot >= a.nq * a.k) return;
    const int lane = threadIdx.x & 63;
    const int64_t q = slot / a.k;
    const int idx = a.top[slot];
    const bool ok = idx >= 0 && (int64_t)idx < a.n;
    if (!ok && lane == 0) report_gather_error(a.err, slot, idx);
    const int64_t row = (a.sets == 1 ? 0 : q * a.n) + (ok ? idx : 0);
    if (a.ids_out && lane == 0) a.ids_out[slot] = (a.ids && ok) ? a.ids[row] : 0;
    uint8_t* dst = a.rows_out + slot * a.row_bytes;
    const uint8_t* src = a.codes + row * a.pitch;
    if ((a.row_bytes & 3) == 0 && (a.pitch & 3) == 0) {
        for (int w = lane; w < a.row_bytes / 4; w += 64)
            ((uint32_t*)dst)[w] = ok ? ((const uint32_t*)src)[w] : 0u;
    } else {
        for (int b = lane; b < a.row_bytes; b += 64) dst[b] = ok ? src[b] : (uint8_t)0;
    }
    uint8_t* sdst = a.scales_out + slot * a.scale_bytes;
    const uint8_t* ssrc = a.scales + row * a.scale_bytes;
    for (int b = lane; b < a.scale_bytes; b += 64) sdst[b] = ok ? ssrc[b] : (uint8_t)0;
}

hipError_t launch_pack_candidates(const PackArgs& a, hipStream_t s) {
    const int64_t slots = a.nq * a.k;
    hipLaunchKernelGGL(pack_candidates_kernel, dim3((unsigned)((slots + 3) / 4)), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace manta
