// kernels_dense.hip -- scores of f32 query vectors against dense f32 / f16
// retrieval vectors with the reference's arithmetic: dotRetrievalVectors
// (runtime/retrieval_eval.go:651-661), `sum += a[i]*b[i]` in f32 over
// i < min(len(a), len(b)), every product and sum rounded on its own (no
// FMA), in index order.
//
// The order of operations is fixed, so the work cannot be reassociated onto
// the matrix cores: each (query, row) pair is one sequential chain of
// v_mul_f32 + v_add_f32.  Throughput comes from running many chains at once:
// a thread owns one row and QB queries (QB independent accumulators), loads
// its row 16 bytes at a time and uses every element QB times; the query
// values are uniform across the workgroup and are read through the scalar
// cache.  Rows of f16 values are widened exactly.  Output: the f32 score
// matrix [nq][n] (the top-k runs on it afterwards).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "device_common.hpp"
#include "kernels.hpp"

#pragma clang fp contract(off)

namespace manta {

namespace {

constexpr int kDenseQB = 8;  // queries per thread

template <typename T>
__device__ __forceinline__ float widen(T x);
template <>
__device__ __forceinline__ float widen<float>(float x) {
    return x;
}
template <>
__device__ __forceinline__ float widen<uint16_t>(uint16_t x) {
    return h2f(x);
}

// VEC: rows are 16-byte aligned and hold whole 16-byte groups of the first
// `len` elements (len * sizeof(T) % 16 == 0 and the row pitch likewise).
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void dense_dot_kernel(const T* __restrict__ rows, int64_t n, int64_t pitch,
                                                        int len, const float* __restrict__ queries, int64_t qpitch,
                                                        int nq, float* __restrict__ out) {
    const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int q0 = blockIdx.y * kDenseQB;
    const int nqb = nq - q0 < kDenseQB ? nq - q0 : kDenseQB;
    if (row >= n) return;
    const T* r = rows + row * pitch;
    const float* qb = queries + (int64_t)q0 * qpitch;
    float acc[kDenseQB];
#pragma unroll
    for (int j = 0; j < kDenseQB; j++) acc[j] = 0.0f;
    constexpr int W = 16 / sizeof(T);  // elements per 16-byte load
    if (VEC) {
        for (int c = 0; c < len; c += W) {
            T v[W];
            *(uint4*)v = *(const uint4*)(r + c);
#pragma unroll
            for (int e = 0; e < W; e++) {
                const float x = widen<T>(v[e]);
#pragma unroll
                for (int j = 0; j < kDenseQB; j++)
                    if (j < nqb) acc[j] = fadd_rn(acc[j], fmul_rn(qb[(int64_t)j * qpitch + c + e], x));
            }
        }
    } else {
        for (int c = 0; c < len; c++) {
            const float x = widen<T>(r[c]);
#pragma unroll
            for (int j = 0; j < kDenseQB; j++)
                if (j < nqb) acc[j] = fadd_rn(acc[j], fmul_rn(qb[(int64_t)j * qpitch + c], x));
        }
    }
#pragma unroll
    for (int j = 0; j < kDenseQB; j++)
        if (j < nqb) out[(int64_t)(q0 + j) * n + row] = acc[j];
}

template <typename T>
hipError_t launch_dense_dot_t(const T* rows, int64_t n, int64_t pitch, int len, const float* queries,
                              int64_t qpitch, int nq, float* out, hipStream_t s) {
    const dim3 grid((unsigned)((n + 255) / 256), (unsigned)((nq + kDenseQB - 1) / kDenseQB));
    constexpr int W = 16 / sizeof(T);
    const bool vec = len % W == 0 && pitch % W == 0 && ((uintptr_t)rows & 15) == 0;
    if (vec) hipLaunchKernelGGL((dense_dot_kernel<T, true>), grid, dim3(256), 0, s, rows, n, pitch, len, queries,
                                qpitch, nq, out);
    else hipLaunchKernelGGL((dense_dot_kernel<T, false>), grid, dim3(256), 0, s, rows, n, pitch, len, queries,
                            qpitch, nq, out);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_dense_dot(const void* rows, int f16, int64_t n, int64_t pitch, int len, const float* queries,
                            int64_t qpitch, int nq, float* out, hipStream_t s) {
    if (n <= 0 || nq <= 0 || len < 0 || (nq + kDenseQB - 1) / kDenseQB > 65535 || (n + 255) / 256 > 0x7FFFFFFF)
        return hipErrorInvalidValue;
    return f16 ? launch_dense_dot_t<uint16_t>((const uint16_t*)rows, n, pitch, len, queries, qpitch, nq, out, s)
               : launch_dense_dot_t<float>((const float*)rows, n, pitch, len, queries, qpitch, nq, out, s);
}

}  // namespace manta
