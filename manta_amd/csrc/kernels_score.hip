// kernels_score.hip -- packed-candidate scoring for gfx950 (streaming path).
//
// One workgroup (256 threads, 4 waves) scores 256 candidate rows per round
// against one query.  q8 rows are read with coalesced 16-byte loads: L lanes
// cover one row (L*16 contiguous bytes per load), C loads per lane per row,
// so a wave moves 64*16 bytes per load instruction.  The int8 products run
// on v_dot4_i32_i8 with the query codes held in registers; row sums are
// reduced across the L lanes with xor shuffles and then transposed so that
// thread t owns row t of the round.  The epilogue computes the exact f32
// score of the packed contract and either stores it (score matrix) or feeds
// the workgroup top-k reservoir (fused top-k; only k keys per workgroup
// reach HBM).
//
// Score formulas (the CPU oracle restates them; reference semantics they
// stand in for: dotRows / cosineRows / l2DistanceRows,
// runtime/backend/tensor_ops.go:1366-1490):
//   q8 dot    (E8 query codes):  t = s_r*acc; t = t*qmax; score = t/127
//   q8 cosine (E16 hi/lo codes): qd = (s_r*qs)*f32(acc); den = |q|*|d_r|;
//                                score = den == 0 ? 0 : qd/den
//   q8 l2     (E16):             score = sqrt(max(0, (qq + dd_r) - 2*qd))
//   q4        (E16):             qd = qs * fma-chain over blocks of
//                                f16scale_b * f32(acc_b); then as above.
#include "device_common.hpp"
#include "kernels.hpp"

namespace manta {


// ------------------------------------------------------------ query codes

// One workgroup per query.  E8 (q8 dot): qmax = max(1, maxabs), code =
// clamp(round((q*127)/qmax)).  E16: code = clamp(round(q*(32639/maxabs))),
// split as code = 256*hi + lo with lo the signed low byte.  Padding columns
// [d, pitch) get code 0.
__global__ __launch_bounds__(256) void query_encode_kernel(
    const uint16_t* __restrict__ q, int d, int pitch, int e16, int8_t* __restrict__ c8,
    int8_t* __restrict__ hi, int8_t* __restrict__ lo, QConst* __restrict__ qc) {
    __shared__ float red_f[256];
    __shared__ long long red_i[256];
    const int qi = blockIdx.x;
    const int tid = threadIdx.x;
    const uint16_t* qrow = q + (int64_t)qi * d;
    float m = 0.0f;
    for (int c = tid; c < d; c += 256) m = fmaxf(m, __builtin_fabsf(h2f(qrow[c])));
    red_f[tid] = m;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s) red_f[tid] = fmaxf(red_f[tid], red_f[tid + s]);
        __syncthreads();
    }
    const float maxabs = red_f[0];
    if (!e16) {
        const float qmax = fmaxf(1.0f, maxabs);
        for (int c = tid; c < pitch; c += 256) {
            float r = 0.0f;
            if (c < d) {
                r = round_half_away(fdiv_rn(fmul_rn(h2f(qrow[c]), 127.0f), qmax));
                r = fminf(127.0f, fmaxf(-127.0f, r));
            }
            c8[(int64_t)qi * pitch + c] = (int8_t)(int)r;
        }
        if (tid == 0) qc[qi] = QConst{qmax, 0.0f, 0.0f, 0.0f};
        return;
    }
    long long ss = 0;
    const float inv = maxabs == 0.0f ? 0.0f : fdiv_rn(32639.0f, maxabs);
    for (int c = tid; c < pitch; c += 256) {
        int code = 0;
        if (c < d && maxabs != 0.0f) {
            float r = round_half_away(fmul_rn(h2f(qrow[c]), inv));
            r = fminf(32639.0f, fmaxf(-32639.0f, r));
            code = (int)r;
        }
        int l = (int)(int8_t)(code & 0xFF);
        int h = (code - l) >> 8;
        hi[(int64_t)qi * pitch + c] = (int8_t)h;
        lo[(int64_t)qi * pitch + c] = (int8_t)l;
        ss += (long long)code * code;
    }
    red_i[tid] = ss;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s) red_i[tid] += red_i[tid + s];
        __syncthreads();
    }
    if (tid == 0) {
        QConst k{0.0f, 0.0f, 0.0f, 0.0f};
        if (maxabs != 0.0f) {
            float qs = fdiv_rn(maxabs, 32639.0f);
            double dss = (double)red_i[0];
            k.a = qs;
            k.b = (float)__dmul_rn(__dsqrt_rn(dss), (double)qs);
            k.c = (float)__dmul_rn(__dmul_rn(dss, (double)qs), (double)qs);
        }
        qc[qi] = k;
    }
}

// ----------------------------------------------------------- epilogues

template <int OP>
__device__ __forceinline__ float q8_epilogue(int acc_or_hi, int lo, float scale, const QConst& k,
                                             float dnorm, float dd) {
    if (OP == OP_DOT) {
        float t = fmul_rn(scale, (float)acc_or_hi);
        t = fmul_rn(t, k.a);
        return fdiv_rn(t, 127.0f);
    }
    // f32(256*hi + lo) with one rounding: both terms are exact in f32.
    float dotf = __fmaf_rn(256.0f, (float)acc_or_hi, (float)lo);
    float qd = fmul_rn(fmul_rn(scale, k.a), dotf);
    if (OP == OP_COSINE) {
        float den = fmul_rn(k.b, dnorm);
        return den == 0.0f ? 0.0f : fdiv_rn(qd, den);
    }
    float t = fadd_rn(k.c, dd);
    float dist2 = fsub_rn(t, fmul_rn(2.0f, qd));
    dist2 = dist2 < 0.0f ? 0.0f : dist2;
    return fsqrt_rn(dist2);
}

template <int OP>
__device__ __forceinline__ float q4_finish(float dotf, const QConst& k, float dnorm, float dd) {
    float qd = fmul_rn(dotf, k.a);
    if (OP == OP_DOT) return qd;
    if (OP == OP_COSINE) {
        float den = fmul_rn(k.b, dnorm);
        return den == 0.0f ? 0.0f : fdiv_rn(qd, den);
    }
    float t = fadd_rn(k.c, dd);
    float dist2 = fsub_rn(t, fmul_rn(2.0f, qd));
    dist2 = dist2 < 0.0f ? 0.0f : dist2;
    return fsqrt_rn(dist2);
}

__device__ __forceinline__ int dot16(v4i a, v4i b, int acc) {
    acc = __builtin_amdgcn_sdot4(a.x, b.x, acc, false);
    acc = __builtin_amdgcn_sdot4(a.y, b.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a.z, b.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a.w, b.w, acc, false);
    return acc;
}

// Common tail of a round: store the score, or offer it to the reservoir.
__device__ __forceinline__ void emit_round(float score, bool valid, int64_t row, int64_t n, int qi,
                                           float* __restrict__ out_scores, uint64_t* keys,
                                           TopKShared* st, uint64_t tau, int smallest) {
    if (out_scores) {
        if (valid) out_scores[(int64_t)qi * n + row] = score;
        return;
    }
    uint64_t key = valid ? make_key(score, (uint32_t)row, smallest) : 0ull;
    topk_offer(key, tau, keys, st);
}



// -------------------------------------------------- q8, coalesced lanes

template <int OP, int L, int C>
__global__ __launch_bounds__(256) void q8_scan_kernel(ScanArgs a) {
    extern __shared__ uint64_t topk_keys[];
    __shared__ TopKShared st;
    constexpr int G = 64 / L;  // rows per wave per load step
    const int qi = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int p = lane % L;
    const int g = lane / L;
    const int64_t set_row0 = (int64_t)qi * a.set_stride;
    const int8_t* __restrict__ codes = a.codes + set_row0 * a.pitch;
    const float* __restrict__ scales = (const float*)a.scales + set_row0;
    const QConst kq = a.qconst[qi];

    v4i qa[C], qb[C];
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int off = c * 16 * L + p * 16;
        if (OP == OP_DOT) {
            qa[c] = *(const v4i*)(a.qc8 + (int64_t)qi * a.pitch + off);
            qb[c] = qa[c];
        } else {
            qa[c] = *(const v4i*)(a.qhi + (int64_t)qi * a.pitch + off);
            qb[c] = *(const v4i*)(a.qlo + (int64_t)qi * a.pitch + off);
        }
    }
    if (!a.out_scores) topk_init(topk_keys, &st);

    const int64_t wg_row0 = (int64_t)blockIdx.x * a.rounds * 256;
    for (int r = 0; r < a.rounds; r++) {
        const int64_t row_base = wg_row0 + (int64_t)r * 256 + wave * 64;
        v4i v[L][C];
#pragma unroll
        for (int it = 0; it < L; it++) {
            const int64_t row = row_base + it * G + g;
#pragma unroll
            for (int c = 0; c < C; c++) {
                if (row < a.n)
                    v[it][c] = __builtin_nontemporal_load(
                        (const v4i*)(codes + row * a.pitch + c * 16 * L + p * 16));
                else
                    v[it][c] = v4i{0, 0, 0, 0};
            }
        }
        int my_hi = 0, my_lo = 0;
#pragma unroll
        for (int it = 0; it < L; it++) {
            int s_hi = 0, s_lo = 0;
#pragma unroll
            for (int c = 0; c < C; c++) {
                s_hi = dot16(v[it][c], qa[c], s_hi);
                if (OP != OP_DOT) s_lo = dot16(v[it][c], qb[c], s_lo);
            }
#pragma unroll
            for (int off = L / 2; off >= 1; off >>= 1) {
                s_hi += __shfl_xor(s_hi, off);
                if (OP != OP_DOT) s_lo += __shfl_xor(s_lo, off);
            }
            const int src = (lane % G) * L;
            int t_hi = __shfl(s_hi, src);
            int t_lo = (OP != OP_DOT) ? __shfl(s_lo, src) : 0;
            if (lane / G == it) {
                my_hi = t_hi;
                my_lo = t_lo;
            }
        }
        const int64_t row = row_base + lane;
        const bool valid = row < a.n;
        float score = 0.0f;
        if (valid) {
            float dn = 0.0f, d2 = 0.0f;
            if (OP == OP_COSINE) dn = a.dnorm[set_row0 + row];
            if (OP == OP_L2) d2 = a.dd[set_row0 + row];
            score = q8_epilogue<OP>(my_hi, my_lo, scales[row], kq, dn, d2);
        }
        uint64_t tau = a.out_scores ? 0ull : st.tau;
        emit_round(score, valid, row, a.n, qi, a.out_scores, topk_keys, &st, tau, a.smallest);
        if (!a.out_scores) {
            __syncthreads();
            topk_maybe_compact(topk_keys, &st, a.k, a.cap);
        }
    }
    if (!a.out_scores) {
        topk_compact(topk_keys, &st, a.k);
        uint64_t* dst = a.partial + ((int64_t)qi * gridDim.x + blockIdx.x) * a.k;
        for (int i = threadIdx.x; i < a.k; i += blockDim.x) dst[i] = i < st.cnt ? topk_keys[i] : 0ull;
    }
}

// --------------------------------------------- q8, any pitch (lane = row)

template <int OP>
__global__ __launch_bounds__(256) void q8_scan_generic_kernel(ScanArgs a) {
    extern __shared__ uint64_t topk_keys[];
    __shared__ TopKShared st;
    const int qi = blockIdx.y;
    const int64_t set_row0 = (int64_t)qi * a.set_stride;
    const int8_t* __restrict__ codes = a.codes + set_row0 * a.pitch;
    const float* __restrict__ scales = (const float*)a.scales + set_row0;
    const QConst kq = a.qconst[qi];
    const int8_t* qa = (OP == OP_DOT ? a.qc8 : a.qhi) + (int64_t)qi * a.pitch;
    const int8_t* qb = a.qlo + (int64_t)qi * a.pitch;
    const int chunks = a.pitch / 16;
    if (!a.out_scores) topk_init(topk_keys, &st);
    const int64_t wg_row0 = (int64_t)blockIdx.x * a.rounds * 256;
    for (int r = 0; r < a.rounds; r++) {
        const int64_t row = wg_row0 + (int64_t)r * 256 + threadIdx.x;
        const bool valid = row < a.n;
        int s_hi = 0, s_lo = 0;
        if (valid) {
            const v4i* rp = (const v4i*)(codes + row * a.pitch);
            for (int c = 0; c < chunks; c++) {
                v4i v = rp[c];
                s_hi = dot16(v, *(const v4i*)(qa + c * 16), s_hi);
                if (OP != OP_DOT) s_lo = dot16(v, *(const v4i*)(qb + c * 16), s_lo);
            }
        }
        float score = 0.0f;
        if (valid) {
            float dn = 0.0f, d2 = 0.0f;
            if (OP == OP_COSINE) dn = a.dnorm[set_row0 + row];
            if (OP == OP_L2) d2 = a.dd[set_row0 + row];
            score = q8_epilogue<OP>(s_hi, s_lo, scales[row], kq, dn, d2);
        }
        uint64_t tau = a.out_scores ? 0ull : st.tau;
        emit_round(score, valid, row, a.n, qi, a.out_scores, topk_keys, &st, tau, a.smallest);
        if (!a.out_scores) {
            __syncthreads();
            topk_maybe_compact(topk_keys, &st, a.k, a.cap);
        }
    }
    if (!a.out_scores) {
        topk_compact(topk_keys, &st, a.k);
        uint64_t* dst = a.partial + ((int64_t)qi * gridDim.x + blockIdx.x) * a.k;
        for (int i = threadIdx.x; i < a.k; i += blockDim.x) dst[i] = i < st.cnt ? topk_keys[i] : 0ull;
    }
}

// ------------------------------------------------------- q4 (lane = row)

// Nibbles to 16x-scaled int8 lanes: (w << 4) & 0xF0F0F0F0 holds the even
// nibbles of w as 16*code, w & 0xF0F0F0F0 the odd ones.  The query digits
// for q4 are stored permuted to match: per 8 columns, [c0 c2 c4 c6] then
// [c1 c3 c5 c7].  Sums are 16x the true block sums and are divided back
// exactly.
template <int OP>
__global__ __launch_bounds__(256) void q4_scan_kernel(ScanArgs a) {
    extern __shared__ uint64_t topk_keys[];
    __shared__ TopKShared st;
    const int qi = blockIdx.y;
    const int64_t set_row0 = (int64_t)qi * a.set_stride;
    const uint8_t* __restrict__ packed = (const uint8_t*)a.codes + set_row0 * a.pitch;
    const uint16_t* __restrict__ scales = (const uint16_t*)a.scales + set_row0 * a.nb;
    const QConst kq = a.qconst[qi];
    // permuted digits: 2*D bytes per digit plane, see host-side permutation
    const int* qh = (const int*)(a.qhi + (int64_t)qi * a.pitch * 2);
    const int* ql = (const int*)(a.qlo + (int64_t)qi * a.pitch * 2);
    if (!a.out_scores) topk_init(topk_keys, &st);
    const int64_t wg_row0 = (int64_t)blockIdx.x * a.rounds * 256;
    for (int r = 0; r < a.rounds; r++) {
        const int64_t row = wg_row0 + (int64_t)r * 256 + threadIdx.x;
        const bool valid = row < a.n;
        float dotf = 0.0f;
        if (valid) {
            const v4i* rp = (const v4i*)(packed + row * a.pitch);
            const uint16_t* sr = scales + row * a.nb;
            for (int b = 0; b < a.nb; b++) {
                v4i w = rp[b];
                int sh = 0, sl = 0;
                int ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    int even = (ws[j] << 4) & (int)0xF0F0F0F0;
                    int odd = ws[j] & (int)0xF0F0F0F0;
                    const int base = b * 8 + j * 2;
                    sh = __builtin_amdgcn_sdot4(even, qh[base], sh, false);
                    sh = __builtin_amdgcn_sdot4(odd, qh[base + 1], sh, false);
                    sl = __builtin_amdgcn_sdot4(even, ql[base], sl, false);
                    sl = __builtin_amdgcn_sdot4(odd, ql[base + 1], sl, false);
                }
                // block sum = (256*sh + sl) / 16, exact
                int acc = (sh * 16) + (sl >> 4);
                dotf = __fmaf_rn(h2f(sr[b]), (float)acc, dotf);
            }
        }
        float score = 0.0f;
        if (valid) {
            float dn = 0.0f, d2 = 0.0f;
            if (OP == OP_COSINE) dn = a.dnorm[set_row0 + row];
            if (OP == OP_L2) d2 = a.dd[set_row0 + row];
            score = q4_finish<OP>(dotf, kq, dn, d2);
        }
        uint64_t tau = a.out_scores ? 0ull : st.tau;
        emit_round(score, valid, row, a.n, qi, a.out_scores, topk_keys, &st, tau, a.smallest);
        if (!a.out_scores) {
            __syncthreads();
            topk_maybe_compact(topk_keys, &st, a.k, a.cap);
        }
    }
    if (!a.out_scores) {
        topk_compact(topk_keys, &st, a.k);
        uint64_t* dst = a.partial + ((int64_t)qi * gridDim.x + blockIdx.x) * a.k;
        for (int i = threadIdx.x; i < a.k; i += blockDim.x) dst[i] = i < st.cnt ? topk_keys[i] : 0ull;
    }
}

// Permute E16 digits for the q4 kernel: per group of 8 columns write
// [c0 c2 c4 c6 c1 c3 c5 c7].  Source and destination planes are [nq][pitch2]
// where pitch2 = d (one byte per column).
__global__ void q4_permute_digits_kernel(const int8_t* __restrict__ src, int8_t* __restrict__ dst,
                                         int d, int64_t total) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    int64_t row = i / d;
    int c = (int)(i % d);
    int grp = c / 8, w = c % 8;
    int srcc = grp * 8 + (w < 4 ? 2 * w : 2 * (w - 4) + 1);
    dst[row * d + c] = src[row * d + srcc];
}

// ------------------------------------------------ exact accumulator rescore

// One thread per selected (query, slot): recompute the q8 integer
// accumulator of the chosen row (E8 for dot, E16 hi/lo combined for the
// others) and write it as int64.
__global__ void q8_rescore_acc_kernel(const int8_t* __restrict__ codes, int pitch, int64_t set_stride,
                                      int64_t n, const int32_t* __restrict__ ids, int k, int nq, int e16,
                                      const int8_t* __restrict__ qc8, const int8_t* __restrict__ qhi,
                                      const int8_t* __restrict__ qlo, int64_t* __restrict__ out) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nq * k) return;
    int qi = i / k;
    int64_t row = ids[i];
    if (row < 0 || row >= n) {
        out[i] = 0;
        return;
    }
    const int8_t* rp = codes + ((int64_t)qi * set_stride + row) * pitch;
    int64_t acc = 0;
    if (!e16) {
        const int8_t* qp = qc8 + (int64_t)qi * pitch;
        for (int c = 0; c < pitch; c++) acc += (int64_t)rp[c] * qp[c];
    } else {
        const int8_t* hp = qhi + (int64_t)qi * pitch;
        const int8_t* lp = qlo + (int64_t)qi * pitch;
        for (int c = 0; c < pitch; c++) acc += (int64_t)rp[c] * (256 * (int64_t)hp[c] + lp[c]);
    }
    out[i] = acc;
}

// ----------------------------------------------------------------- hosts

hipError_t launch_query_encode(const uint16_t* q, int nq, int d, int pitch, int e16, int8_t* c8,
                               int8_t* hi, int8_t* lo, QConst* qc, hipStream_t s) {
    hipLaunchKernelGGL(query_encode_kernel, dim3(nq), dim3(256), 0, s, q, d, pitch, e16, c8, hi,
                       lo, qc);
    return hipGetLastError();
}

hipError_t launch_q4_permute(const int8_t* src, int8_t* dst, int d, int nq, hipStream_t s) {
    int64_t total = (int64_t)nq * d;
    hipLaunchKernelGGL(q4_permute_digits_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                       0, s, src, dst, d, total);
    return hipGetLastError();
}

template <int OP>
static hipError_t launch_q8_op(const ScanArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    const int chunks = a.pitch / 16;
#define MANTA_Q8(LL, CC)                                                               \
    if (chunks == (LL) * (CC)) {                                                       \
        hipLaunchKernelGGL((q8_scan_kernel<OP, LL, CC>), grid, dim3(256), lds, s, a); \
        return hipGetLastError();                                                      \
    }
    MANTA_Q8(4, 1)    // d <= 64
    MANTA_Q8(8, 1)    // 128
    MANTA_Q8(4, 3)    // 192
    MANTA_Q8(16, 1)   // 256
    MANTA_Q8(8, 3)    // 384
    MANTA_Q8(16, 2)   // 512
    MANTA_Q8(16, 3)   // 768
    MANTA_Q8(16, 4)   // 1024
#undef MANTA_Q8
    hipLaunchKernelGGL((q8_scan_generic_kernel<OP>), grid, dim3(256), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_q8_scan(int op, const ScanArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    switch (op) {
        case OP_DOT: return launch_q8_op<OP_DOT>(a, grid, lds, s);
        case OP_COSINE: return launch_q8_op<OP_COSINE>(a, grid, lds, s);
        default: return launch_q8_op<OP_L2>(a, grid, lds, s);
    }
}

hipError_t launch_q4_scan(int op, const ScanArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    switch (op) {
        case OP_DOT: hipLaunchKernelGGL((q4_scan_kernel<OP_DOT>), grid, dim3(256), lds, s, a); break;
        case OP_COSINE: hipLaunchKernelGGL((q4_scan_kernel<OP_COSINE>), grid, dim3(256), lds, s, a); break;
        default: hipLaunchKernelGGL((q4_scan_kernel<OP_L2>), grid, dim3(256), lds, s, a); break;
    }
    return hipGetLastError();
}

hipError_t launch_q8_rescore(const int8_t* codes, int pitch, int64_t set_stride, int64_t n,
                             const int32_t* ids, int k, int nq, int e16, const int8_t* qc8,
                             const int8_t* qhi, const int8_t* qlo, int64_t* out, hipStream_t s) {
    int total = nq * k;
    hipLaunchKernelGGL(q8_rescore_acc_kernel, dim3((total + 127) / 128), dim3(128), 0, s, codes,
                       pitch, set_stride, n, ids, k, nq, e16, qc8, qhi, qlo, out);
    return hipGetLastError();
}

}  // namespace manta
