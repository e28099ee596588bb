// kernels_encoder.hip -- device steps of the encoder pipeline (gather of q8
// token rows, f32 MFMA GEMMs with fused q8 column dequant, row softmax,
// residual add + layernorm, gelu), composed by manta_rocm_encoder_pooled.
//
// All arithmetic is f32 (f64 where the reference uses it: the softmax sum
// and exponentials, the layernorm's reciprocal square root, gelu's tanh).
// Reductions run in tree order, so results match the reference's
// sequential loops within rounding, not bit for bit.
#include "device_common.hpp"
#include "kernels.hpp"

namespace manta {

namespace {

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

}  // namespace

// X[i][c] = codes[tok[i]][c] * scale[tok[i]] (f32); an id out of range is
// recorded in err (flag | id) and its row is zero.
__global__ __launch_bounds__(256) void enc_gather_q8_kernel(const int32_t* __restrict__ tok, int64_t rows,
                                                            const int8_t* __restrict__ codes,
                                                            const float* __restrict__ scales, int64_t vocab, int d,
                                                            float* __restrict__ x, unsigned long long* err,
                                                            uint16_t* __restrict__ x16) {
    const int64_t total = rows * d;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / d;
        const int c = (int)(i - r * d);
        const int id = tok[r];
        const bool ok = id >= 0 && (int64_t)id < vocab;
        if (!ok && c == 0) report_gather_error(err, r, id);
        const float v = ok ? fmul_rn((float)codes[(int64_t)id * d + c], scales[id]) : 0.0f;
        x[i] = v;
        if (x16) x16[i] = f2h(v);
    }
}

// C[b] = A[b] (M x K, row-major, batch stride sA) times B:
//   BMODE 0: B[b] f32 [K][N] row-major (batch stride sB)
//   BMODE 1: int8 [K][N] with an f32 scale per column (shared), dequantized
//            as code * scale while staging
//   BMODE 2: the transpose of Bm[b], an f32 [N][K] row-major matrix
// on the f32 matrix cores: a 64 x 64 output tile per workgroup as four 32 x 32
// quarters, one per wave, each accumulated by v_mfma_f32_32x32x2f32 (lane l
// supplies A[m = l%32][k = l/32] and B[k = l/32][n = l%32]; result row
// 8*(r/4) + 4*(l/32) + r%4, column l%32 of its 16 values).  K moves in steps
// of 16 through LDS; grid = (tiles of N, tiles of M, batches).  gelu != 0
// applies geluTensor to each output value before the store (the FFN's
// up-projection), the same f32 result as a separate pass.
template <int BMODE, bool VEC>
__global__ __launch_bounds__(256) void enc_gemm_mfma_kernel(const float* __restrict__ A, int64_t sA,
                                                            const void* __restrict__ Bv,
                                                            const float* __restrict__ bscale, int64_t sB,
                                                            float* __restrict__ C, int64_t sC, int M, int N, int K,
                                                            int gelu, uint16_t* __restrict__ C16) {
    typedef float v16f __attribute__((ext_vector_type(16)));
    __shared__ float As[16][64 + 4];
    __shared__ float Bs[16][64 + 4];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const int64_t bt = blockIdx.z;
    const float* a = A + bt * sA;
    v16f acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += 16) {
        if (VEC) {
            // one 16-byte load per thread per tile (K % 16 == 0; N % 4 == 0
            // unless B is transposed): A by 4 consecutive k of a row
            {
                const int m = tid >> 2, kq = (tid & 3) * 4;
                const int gm = m0 + m;
                const float4 v = gm < M ? *(const float4*)(a + (int64_t)gm * K + k0 + kq) : float4{0, 0, 0, 0};
                As[kq][m] = v.x, As[kq + 1][m] = v.y, As[kq + 2][m] = v.z, As[kq + 3][m] = v.w;
            }
            if (BMODE == 2) {
                const int n = tid >> 2, kq = (tid & 3) * 4;
                const int gn = n0 + n;
                const float4 v = gn < N ? *(const float4*)((const float*)Bv + bt * sB + (int64_t)gn * K + k0 + kq)
                                        : float4{0, 0, 0, 0};
                Bs[kq][n] = v.x, Bs[kq + 1][n] = v.y, Bs[kq + 2][n] = v.z, Bs[kq + 3][n] = v.w;
            } else {
                const int kk = tid >> 4, nq = (tid & 15) * 4;
                const int gn = n0 + nq;
                float4 v = {0, 0, 0, 0};
                if (gn < N) {
                    const int64_t off = (int64_t)(k0 + kk) * N + gn;
                    if (BMODE == 0) {
                        v = *(const float4*)((const float*)Bv + bt * sB + off);
                    } else {
                        const char4 c = *(const char4*)((const int8_t*)Bv + off);
                        const float4 sc = *(const float4*)(bscale + gn);
                        v = float4{fmul_rn((float)c.x, sc.x), fmul_rn((float)c.y, sc.y), fmul_rn((float)c.z, sc.z),
                                   fmul_rn((float)c.w, sc.w)};
                    }
                }
                *(float4*)&Bs[kk][nq] = v;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int e = tid + 256 * i;
                const int m = e >> 4, kk = e & 15;
                const int gm = m0 + m, gk = k0 + kk;
                As[kk][m] = (gm < M && gk < K) ? a[(int64_t)gm * K + gk] : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int e = tid + 256 * i;
                float v = 0.0f;
                if (BMODE == 2) {
                    const int n = e >> 4, kk = e & 15;
                    const int gn = n0 + n, gk = k0 + kk;
                    if (gn < N && gk < K) v = ((const float*)Bv)[bt * sB + (int64_t)gn * K + gk];
                    Bs[kk][n] = v;
                } else {
                    const int kk = e >> 6, n = e & 63;
                    const int gn = n0 + n, gk = k0 + kk;
                    if (gn < N && gk < K) {
                        if (BMODE == 0) v = ((const float*)Bv)[bt * sB + (int64_t)gk * N + gn];
                        else v = fmul_rn((float)((const int8_t*)Bv)[(int64_t)gk * N + gn], bscale[gn]);
                    }
                    Bs[kk][n] = v;
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; kk += 2) {
            const float av = As[kk + (lane >> 5)][wm + (lane & 31)];
            const float bv = Bs[kk + (lane >> 5)][wn + (lane & 31)];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc, 0, 0, 0);
        }
        __syncthreads();
    }
    float* c = C + bt * sC;
    const int gn = n0 + wn + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int gm = m0 + wm + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (gm < M && gn < N) {
            const float v = gelu ? gelu_value(acc[r]) : acc[r];
            c[(int64_t)gm * N + gn] = v;
            if (C16) C16[bt * sC + (int64_t)gm * N + gn] = f2h(v);
        }
    }
}

// Row softmax in place (softmaxRows): one wave per row.
__global__ __launch_bounds__(256) void enc_softmax_rows_kernel(float* __restrict__ x, int64_t rows, int cols) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    float* row = x + r * cols;
    float m = -__builtin_inff();
    for (int c = lane; c < cols; c += 64) m = fmaxf(m, row[c]);
    m = wave_max_f32(m);
    double s = 0.0;
    for (int c = lane; c < cols; c += 64) {
        const double ev = exp((double)fsub_rn(row[c], m));
        row[c] = (float)ev;
        s += ev;
    }
    s = wave_sum_f64(s);
    if (s == 0.0) return;
    const float inv = (float)(1.0 / s);
    for (int c = lane; c < cols; c += 64) row[c] = fmul_rn(row[c], inv);
}

// y = layernorm(a + b) per row (binary_add then layerNormRows): one wave per
// row; f32 mean and variance, f64 reciprocal square root of variance + 1e-5.
// ADD false: layerNormRows(a) alone (b unused).
template <bool ADD>
__global__ __launch_bounds__(256) void enc_add_layernorm_kernel(const float* __restrict__ a,
                                                                const float* __restrict__ b, float* __restrict__ y,
                                                                int64_t rows, int cols, uint16_t* __restrict__ y16) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float* ar = a + r * cols;
    const float* br = ADD ? b + r * cols : nullptr;
    float* yr = y + r * cols;
    auto in = [&](int c) { return ADD ? fadd_rn(ar[c], br[c]) : ar[c]; };
    float s = 0.0f;
    for (int c = lane; c < cols; c += 64) s = fadd_rn(s, in(c));
    const float mean = fdiv_rn(wave_sum_f32(s), (float)cols);
    float v = 0.0f;
    for (int c = lane; c < cols; c += 64) {
        const float d = fsub_rn(in(c), mean);
        v = __fmaf_rn(d, d, v);
    }
    const float var = fdiv_rn(wave_sum_f32(v), (float)cols);
    const float inv = (float)(1.0 / sqrt((double)var + 1e-5));
    for (int c = lane; c < cols; c += 64) {
        const float o = fmul_rn(fsub_rn(in(c), mean), inv);
        yr[c] = o;
        if (y16) y16[r * cols + c] = f2h(o);
    }
}

// geluTensor in place, element by element.
__global__ __launch_bounds__(256) void enc_gelu_kernel(float* __restrict__ x, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        x[i] = gelu_value(x[i]);
}

__global__ __launch_bounds__(256) void enc_to_f16_kernel(const float* __restrict__ x, int64_t n,
                                                         uint16_t* __restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        out[i] = f2h(x[i]);
}

static unsigned grid_for(int64_t n) {
    const int64_t g = (n + 255) / 256;
    return (unsigned)(g < 65536 ? (g < 1 ? 1 : g) : 65536);
}

hipError_t launch_enc_gather_q8(const int32_t* tok, int64_t rows, const int8_t* codes, const float* scales,
                                int64_t vocab, int d, float* x, unsigned long long* err, hipStream_t s,
                                uint16_t* x16) {
    hipLaunchKernelGGL(enc_gather_q8_kernel, dim3(grid_for(rows * d)), dim3(256), 0, s, tok, rows, codes, scales,
                       vocab, d, x, err, x16);
    return hipGetLastError();
}

hipError_t launch_enc_gemm(int bmode, const float* A, int64_t sA, const void* B, const float* bscale, int64_t sB,
                           float* C, int64_t sC, int M, int N, int K, int batches, hipStream_t s, bool gelu,
                           uint16_t* C16) {
    if (M <= 0 || N <= 0 || K <= 0 || batches <= 0 || batches > 65535 || (M + 63) / 64 > 65535)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64), (unsigned)batches);
    // 16-byte staging loads need whole K steps and 16-byte aligned rows (the
    // batch strides and base pointers are multiples of 4 elements here)
    const bool vec = K % 16 == 0 && (bmode == 2 || N % 4 == 0) && sA % 4 == 0 && sB % 4 == 0 &&
                     ((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0 && (bmode != 1 || ((uintptr_t)bscale & 15) == 0);
#define MANTA_ENC_GEMM(BM)                                                                                      \
    do {                                                                                                        \
        if (vec)                                                                                                \
            hipLaunchKernelGGL((enc_gemm_mfma_kernel<BM, true>), grid, dim3(256), 0, s, A, sA, B, bscale, sB, C, \
                               sC, M, N, K, gelu ? 1 : 0, C16);                                                               \
        else                                                                                                    \
            hipLaunchKernelGGL((enc_gemm_mfma_kernel<BM, false>), grid, dim3(256), 0, s, A, sA, B, bscale, sB,   \
                               C, sC, M, N, K, gelu ? 1 : 0, C16);                                                            \
    } while (0)
    if (bmode == 0) MANTA_ENC_GEMM(0);
    else if (bmode == 1) MANTA_ENC_GEMM(1);
    else MANTA_ENC_GEMM(2);
#undef MANTA_ENC_GEMM
    return hipGetLastError();
}

hipError_t launch_enc_softmax_rows(float* x, int64_t rows, int cols, hipStream_t s) {
    hipLaunchKernelGGL(enc_softmax_rows_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, x, rows, cols);
    return hipGetLastError();
}

hipError_t launch_enc_add_layernorm(const float* a, const float* b, float* y, int64_t rows, int cols,
                                    hipStream_t s, uint16_t* y16) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    if (b)
        hipLaunchKernelGGL(enc_add_layernorm_kernel<true>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, a, b, y,
                           rows, cols, y16);
    else
        hipLaunchKernelGGL(enc_add_layernorm_kernel<false>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, a, b,
                           y, rows, cols, y16);
    return hipGetLastError();
}

hipError_t launch_enc_gelu(float* x, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(enc_gelu_kernel, dim3(grid_for(n)), dim3(256), 0, s, x, n);
    return hipGetLastError();
}


hipError_t launch_enc_to_f16(const float* x, int64_t n, uint16_t* out, hipStream_t s) {
    hipLaunchKernelGGL(enc_to_f16_kernel, dim3(grid_for(n)), dim3(256), 0, s, x, n, out);
    return hipGetLastError();
}

}  // namespace manta
