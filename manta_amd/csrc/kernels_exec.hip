// kernels_exec.hip -- the small device steps the artifact executor needs
// besides the scoring, top-k and embed kernels:
//
//   gather_elems  gatherTensor (tensor_ops.go:751-979) for dense tables of
//                 2-, 4- or 8-byte elements, every table-rank x index-rank
//                 case as one copy: out[(b*K + i)*C + c] =
//                 table[b*bstride + idx[b*K + i]*C + c];
//   widen_f16     binary16 -> f32 (exact), for f16 values fed to f32 steps;
//   mean_pool     meanPoolTensor (tensor_ops.go:1170-1208): f32 sums in
//                 position order divided by float32(T) (a true division, not
//                 the masked form's multiplication by 1/count).
//
// All three are bandwidth-bound copies or sums: one element per thread,
// consecutive threads on consecutive elements of a row.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "device_common.hpp"
#include "kernels.hpp"

namespace manta {

namespace {

template <typename T>
__global__ __launch_bounds__(256) void gather_elems_kernel(const T* __restrict__ table, int64_t rows, int64_t cols,
                                                           int64_t bstride, const int32_t* __restrict__ idx,
                                                           int64_t K, int64_t total, T* __restrict__ out,
                                                           unsigned long long* err) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t slot = i / cols;  // b*K + k: the index position
        const int64_t c = i - slot * cols;
        const int id = idx[slot];
        const bool ok = id >= 0 && (int64_t)id < rows;
        if (!ok && c == 0) report_gather_error(err, slot, id);
        const int64_t b = slot / K;
        out[i] = ok ? table[b * bstride + (int64_t)id * cols + c] : (T)0;
    }
}

__global__ __launch_bounds__(256) void widen_f16_kernel(const uint16_t* __restrict__ in, float* __restrict__ out,
                                                        int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        out[i] = h2f(in[i]);
}

__global__ __launch_bounds__(256) void mean_pool_kernel(const float* __restrict__ x, int64_t B, int64_t T, int64_t C,
                                                        float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= B * C) return;
    const int64_t b = i / C, c = i - b * C;
    float s = 0.0f;
    for (int64_t t = 0; t < T; t++) s = fadd_rn(s, x[(b * T + t) * C + c]);
    out[i] = fdiv_rn(s, (float)T);
}

template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(const T* __restrict__ in, int64_t R, int64_t C, int64_t total,
                                                        T* __restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        // output element i of [B][C][R]: read in[b][r][c]
        const int64_t rc = R * C;
        const int64_t b = i / rc, j = i - b * rc;
        const int64_t c = j / R, r = j - c * R;
        out[i] = in[b * rc + r * C + c];
    }
}

__global__ __launch_bounds__(256) void binary_f32_kernel(int op, const float* __restrict__ a,
                                                         const float* __restrict__ b, float* __restrict__ out,
                                                         int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const float x = a[i], y = b[i];
        out[i] = op == 0 ? fadd_rn(x, y) : op == 1 ? fsub_rn(x, y) : op == 2 ? fmul_rn(x, y) : fdiv_rn(x, y);
    }
}

__global__ __launch_bounds__(256) void dequant_q8_kernel(const int8_t* __restrict__ codes,
                                                         const float* __restrict__ scales, int64_t cols,
                                                         int per_col, int64_t total, float* __restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / cols;
        out[i] = fmul_rn((float)codes[i], scales[per_col ? i - r * cols : r]);
    }
}

unsigned grid_for(int64_t total) {
    const int64_t g = (total + 255) / 256;
    return (unsigned)(g < 65536 * 4 ? (g < 1 ? 1 : g) : 65536 * 4);
}

}  // namespace

hipError_t launch_gather_elems(const void* table, int elem_bytes, int64_t rows, int64_t cols, int64_t bstride,
                               const int32_t* idx, int64_t B, int64_t K, void* out, unsigned long long* err,
                               hipStream_t s) {
    const int64_t total = B * K * cols;
    if (total <= 0) return hipSuccess;
    const unsigned grid = grid_for(total);
    switch (elem_bytes) {
        case 2:
            hipLaunchKernelGGL(gather_elems_kernel<uint16_t>, dim3(grid), dim3(256), 0, s, (const uint16_t*)table,
                               rows, cols, bstride, idx, K, total, (uint16_t*)out, err);
            break;
        case 4:
            hipLaunchKernelGGL(gather_elems_kernel<uint32_t>, dim3(grid), dim3(256), 0, s, (const uint32_t*)table,
                               rows, cols, bstride, idx, K, total, (uint32_t*)out, err);
            break;
        case 8:
            hipLaunchKernelGGL(gather_elems_kernel<uint64_t>, dim3(grid), dim3(256), 0, s, (const uint64_t*)table,
                               rows, cols, bstride, idx, K, total, (uint64_t*)out, err);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_widen_f16(const uint16_t* in, float* out, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(widen_f16_kernel, dim3(grid_for(n)), dim3(256), 0, s, in, out, n);
    return hipGetLastError();
}

hipError_t launch_transpose(const void* in, int elem_bytes, int64_t B, int64_t R, int64_t C, void* out,
                            hipStream_t s) {
    const int64_t total = B * R * C;
    if (total <= 0) return hipSuccess;
    const unsigned grid = grid_for(total);
    switch (elem_bytes) {
        case 2:
            hipLaunchKernelGGL(transpose_kernel<uint16_t>, dim3(grid), dim3(256), 0, s, (const uint16_t*)in, R, C,
                               total, (uint16_t*)out);
            break;
        case 4:
            hipLaunchKernelGGL(transpose_kernel<uint32_t>, dim3(grid), dim3(256), 0, s, (const uint32_t*)in, R, C,
                               total, (uint32_t*)out);
            break;
        case 8:
            hipLaunchKernelGGL(transpose_kernel<uint64_t>, dim3(grid), dim3(256), 0, s, (const uint64_t*)in, R, C,
                               total, (uint64_t*)out);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_binary_f32(int op, const float* a, const float* b, float* out, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(binary_f32_kernel, dim3(grid_for(n)), dim3(256), 0, s, op, a, b, out, n);
    return hipGetLastError();
}

hipError_t launch_dequant_q8(const int8_t* codes, const float* scales, int64_t rows, int64_t cols, int per_col,
                             float* out, hipStream_t s) {
    const int64_t total = rows * cols;
    if (total <= 0) return hipSuccess;
    hipLaunchKernelGGL(dequant_q8_kernel, dim3(grid_for(total)), dim3(256), 0, s, codes, scales, cols, per_col, total,
                       out);
    return hipGetLastError();
}

hipError_t launch_mean_pool(const float* x, int64_t B, int64_t T, int64_t C, float* out, hipStream_t s) {
    const int64_t total = B * C;
    if (total <= 0) return hipSuccess;
    hipLaunchKernelGGL(mean_pool_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, x, B, T, C, out);
    return hipGetLastError();
}

}  // namespace manta
