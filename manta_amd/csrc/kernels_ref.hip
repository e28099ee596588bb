// kernels_ref.hip -- scores with the reference's own arithmetic (dotRows,
// cosineRows, l2DistanceRows; runtime/backend/tensor_ops.go:1366-1490) on the
// values packed q8 / q4 rows stand for.
//
// ref_rescore_kernel (one candidate per thread): the quantized-query scans
// return their best kp rows; each is rescored with the reference arithmetic.
// ref_finish_kernel (one workgroup per query) sorts them by (score, index)
// as topKTensor does
// (tensor_ops.go:1539-1551), and keeps the best k if the bounds of
// ref_common.hpp prove that no row outside the kp can reach the k-th: for
// largest-first, every outside row has a scan score of at most that of the
// kp-th row, c, hence a reference score of at most ref_hi(c), and the proof
// is ref_hi(c) < L with L the k-th best reference score found (smallest-
// first: ref_lo(c) > L).  Otherwise the query is marked for ref_scan.
//
// ref_scan_kernel: lane = row, the reference score of every row; writes the
// score matrix, or feeds the streaming reservoir (device_common.hpp) and the
// last-workgroup merge (scan_common.hpp) for the queries marked by the
// finish, from the threshold key L gives.
#include "device_common.hpp"
#include "kernels.hpp"
#include "mq_common.hpp"
#include "ref_common.hpp"
#include "scan_common.hpp"

namespace manta {

template <int FMT, int OP>
__device__ __forceinline__ float ref_row_score(const void* codes, const void* scales, const double* sqd,
                                               int64_t row, int pitch, int d, const float* qf, double sqn) {
    const double dn = OP == OP_COSINE ? sqd[row] : 0.0;
    if (FMT == 8)
        return ref_score_q8<OP>(qf, (const int8_t*)codes + row * pitch, ((const float*)scales)[row], d, sqn, dn);
    return ref_score_q4<OP>(qf, (const uint8_t*)codes + row * pitch, (const uint16_t*)scales + row * (d / 32), d,
                            sqn, dn);
}

// Keys of the finish: next_pow2(kp) <= kRefMaxKeys in LDS.
constexpr int kRefMaxKeys = 4096;

// Reference keys of the scan's kp candidates of each query: one candidate per
// thread, grid (ceil(kp / 256), nq).  keys [nq][kp] (0 for an invalid id).
template <int FMT, int OP>
__global__ __launch_bounds__(256) void ref_rescore_kernel(RefArgs a, uint64_t* __restrict__ keys) {
    __shared__ float qf[kMaxQueryDim];
    __shared__ double sqn_s;
    const int q = blockIdx.y;
    const int d = a.d;
    const uint16_t* qrow = a.queries + (int64_t)q * d;
    const int i = blockIdx.x * 256 + threadIdx.x;
    const bool has = i < a.kp;
    const int32_t id = has ? a.cand_ids[(int64_t)q * a.kp + i] : -1;
    for (int c = threadIdx.x; c < d; c += 256) qf[c] = h2f(qrow[c]);
    __syncthreads();
    // cosine: the query's f64 norm (a sequential sum) on the last thread,
    // which holds no candidate unless all 256 do, while the others sum theirs
    if (OP == OP_COSINE && threadIdx.x == 255) sqn_s = ref_sqrt_norm(qf, d);
    const bool ok = id >= 0 && (int64_t)id < a.n;
    const int64_t row = (int64_t)q * a.set_stride + (ok ? id : 0);
    RefAcc<OP> acc;
    double dn = 0.0;
    if (ok) {
        if (OP == OP_COSINE) dn = a.sqd[row];
        if (FMT == 8)
            acc = ref_acc_q8<OP>(qf, (const int8_t*)a.codes + row * a.pitch, ((const float*)a.scales)[row], d);
        else
            acc = ref_acc_q4<OP>(qf, (const uint8_t*)a.codes + row * a.pitch,
                                 (const uint16_t*)a.scales + row * (d / 32), d);
    }
    if (OP == OP_COSINE) __syncthreads();  // sqn_s is published
    if (!has) return;
    const double sqn = OP == OP_COSINE ? sqn_s : 0.0;
    keys[(int64_t)q * a.kp + i] = ok ? make_key(acc.finish(sqn, dn), (uint32_t)id, a.smallest) : 0ull;
}

// One workgroup per query: sort the candidates' reference keys, take the
// k-th, and prove (or not) from the scan score of the kp-th candidate that
// no other row reaches it.
template <int OP, int NT>
__global__ __launch_bounds__(NT) void ref_finish_kernel(RefArgs a, const uint64_t* __restrict__ cand_keys) {
    constexpr int NW = NT / 64;
    extern __shared__ uint64_t keys[];
    __shared__ float red_m[NW];
    __shared__ double red_g[NW], red_n[NW];
    __shared__ long long red_s[NW];
    __shared__ int ok_s;
    const int q = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int d = a.d;
    const uint16_t* qrow = a.queries + (int64_t)q * d;
    const int kp = a.kp;
    const int S = next_pow2(kp < 2 ? 2 : kp);
    for (int i = tid; i < S; i += NT) keys[i] = i < kp ? cand_keys[(int64_t)q * kp + i] : 0ull;

    // the quantities of the bounds: the scans' E16 codes of the query (same
    // arithmetic as encode_query_block), G = |q - qs*code|, |q|, sum code^2
    float m = 0.0f;
    for (int c = tid; c < d; c += NT) m = fmaxf(m, __builtin_fabsf(h2f(qrow[c])));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (lane == 0) red_m[wave] = m;
    __syncthreads();
    float maxabs = 0.0f;
    for (int w = 0; w < NW; w++) maxabs = fmaxf(maxabs, red_m[w]);
    const float inv = maxabs == 0.0f ? 0.0f : fdiv_rn(32639.0f, maxabs);
    const float qs = maxabs == 0.0f ? 0.0f : fdiv_rn(maxabs, 32639.0f);
    double g2 = 0.0, n2 = 0.0;
    long long ss = 0;
    for (int c = tid; c < d; c += NT) {
        const float x = h2f(qrow[c]);
        const int code = maxabs != 0.0f ? code_e16(x, inv) : 0;
        const double diff = (double)x - (double)code * (double)qs;
        g2 += diff * diff;
        n2 += (double)x * (double)x;
        ss += (long long)code * code;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        g2 += __shfl_xor(g2, off);
        n2 += __shfl_xor(n2, off);
        ss += __shfl_xor(ss, off);
    }
    if (lane == 0) {
        red_g[wave] = g2;
        red_n[wave] = n2;
        red_s[wave] = ss;
    }
    __syncthreads();
    block_sort_desc_regs<NT>(keys, S);

    if (tid == 0) {
        const uint64_t kth = keys[a.k - 1];
        const float L = key_score(kth, a.smallest);
        bool ok = kth != 0;
        if (ok && (int64_t)kp < a.n) {
            if (maxabs == 0.0f && OP != OP_L2) {
                // a zero query: every reference dot / cosine is +0, as every
                // scan score, so the scan's first kp rows hold the k lowest
                ok = true;
            } else {
                const double up = 1.0 + 9.094947017729282e-13;
                double sg = 0.0, sn = 0.0;
                long long sc = 0;
                for (int w = 0; w < NW; w++) {
                    sg += red_g[w];
                    sn += red_n[w];
                    sc += red_s[w];
                }
                const double G = __builtin_sqrt(sg) * up;
                const double qn = __builtin_sqrt(sn) * up;
                const double qh = __builtin_sqrt((double)sc) * (double)qs * up;
                const double wide = 1.0 + 2.384185791015625e-07;  // 1 + 2^-22
                const RefBounds b = ref_bounds(OP, G, qn, qh, (double)a.e_qd, (double)a.maxdn * wide,
                                               (double)a.maxdd * wide, d);
                const double c = (double)a.cand_scores[(int64_t)q * kp + kp - 1];
                ok = b.ok && (a.smallest ? ref_lo(b, c) > (double)L : ref_hi(b, c) < (double)L);
            }
        }
        ok_s = ok ? 1 : 0;
        a.redo[q] = ok ? 0 : 1;
        // every key of the final k is at least kth, hence at least the
        // smallest key of its score (low word 0x7FFFFFFF is below every ~idx)
        a.redo_tau[q] = kth ? make_key(L, 0x80000000u, a.smallest) : 0ull;
    }
    __syncthreads();
    if (!ok_s) return;
    for (int i = tid; i < a.k; i += NT) {
        const uint64_t key = keys[i];
        a.out_ids[(int64_t)q * a.k + i] = key ? (int32_t)key_index(key) : -1;
        if (a.out_scores) a.out_scores[(int64_t)q * a.k + i] = key ? key_score(key, a.smallest) : 0.0f;
    }
}

// Reference scores of every row, lane = row.  Score matrix (a.out_scores):
// grid (parts, nq), one query per blockIdx.y.  Top-k: grid (parts, R); the
// workgroups of blockIdx.y = r take the queries r, r + R, ... the finish
// marked (redo == nullptr: all of them), each with the streaming reservoir
// from the threshold key redo_tau and the last-workgroup merge over the
// gridDim.x parts.  A query nobody marked costs its workgroups one flag read.
template <int FMT, int OP>
__global__ __launch_bounds__(256) void ref_scan_kernel(ScanArgs a, int nq, const double* __restrict__ sqd,
                                                       const int* __restrict__ redo,
                                                       const uint64_t* __restrict__ redo_tau) {
    extern __shared__ uint64_t topk_keys[];
    __shared__ ScanTopkLds S;
    __shared__ float qf[kMaxQueryDim];
    __shared__ double sqn_s;
    __shared__ int marked[256];
    __shared__ int nmarked;
    const bool topk = a.out_scores == nullptr;
    // this slot's queries, 256 at a time: the marks are read in parallel and
    // the marked queries listed in LDS (the list is usually empty)
    const int per_slot = (nq - (int)blockIdx.y + (int)gridDim.y - 1) / (int)gridDim.y;
    for (int base = 0; base < per_slot; base += 256) {
        __syncthreads();  // the previous batch's list is consumed
        if (threadIdx.x == 0) nmarked = 0;
        __syncthreads();
        {
            const int j = base + (int)threadIdx.x;
            const int qj = (int)blockIdx.y + j * (int)gridDim.y;
            if (j < per_slot && (!topk || !redo || redo[qj])) marked[atomicAdd(&nmarked, 1)] = qj;
        }
        __syncthreads();
        const int nm = nmarked;
        for (int mi = 0; mi < nm; mi++) {
            const int qi = marked[mi];
            const uint64_t tau0 = (topk && redo_tau) ? redo_tau[qi] : 0ull;
            __syncthreads();  // the previous query's readers of qf and the reservoir are done
            const uint16_t* qrow = a.queries + (int64_t)qi * a.d;
            for (int c = threadIdx.x; c < a.d; c += 256) qf[c] = h2f(qrow[c]);
            __syncthreads();
            if (OP == OP_COSINE && threadIdx.x == 0) sqn_s = ref_sqrt_norm(qf, a.d);
            if (topk) topk_init(topk_keys, &S.st);  // (its barrier publishes sqn_s)
            else __syncthreads();
            const double sqn = OP == OP_COSINE ? sqn_s : 0.0;
            const int64_t set_row0 = (int64_t)qi * a.set_stride;
            const int64_t wg_row0 = (int64_t)blockIdx.x * a.rounds * 256;
            for (int r = 0; r < a.rounds; r++) {
                const int64_t row = wg_row0 + (int64_t)r * 256 + threadIdx.x;
                const bool valid = row < a.n;
                float s = 0.0f;
                if (valid)
                    s = ref_row_score<FMT, OP>(a.codes, a.scales, sqd, set_row0 + row, a.pitch, a.d, qf, sqn);
                if (!topk) {
                    if (valid) a.out_scores[(int64_t)qi * a.n + row] = s;
                    continue;
                }
                const uint64_t key = valid ? make_key(s, (uint32_t)row, a.smallest) : 0ull;
                const uint64_t tau = S.st.tau > tau0 ? S.st.tau : tau0;
                topk_offer(key, tau, topk_keys, &S.st);
                if (a.mid_compact) {
                    __syncthreads();
                    topk_maybe_compact(topk_keys, &S.st, a.k, a.cap);
                }
            }
            if (topk) finish_topk(a, topk_keys, S, qi);
        }
    }
}

// ----------------------------------------------------------------- hosts

static int next_pow2_host(int x) {
    int p = 2;
    while (p < x) p <<= 1;
    return p;
}

template <int FMT, int OP>
static void launch_ref_rescore_op(const RefArgs& a, uint64_t* keys, hipStream_t s) {
    const dim3 grid((unsigned)((a.kp + 255) / 256), (unsigned)a.nq);
    hipLaunchKernelGGL((ref_rescore_kernel<FMT, OP>), grid, dim3(256), 0, s, a, keys);
}

template <int FMT>
static void launch_ref_rescore_fmt(const RefArgs& a, uint64_t* keys, hipStream_t s) {
    switch (a.op) {
        case OP_DOT: launch_ref_rescore_op<FMT, OP_DOT>(a, keys, s); break;
        case OP_COSINE: launch_ref_rescore_op<FMT, OP_COSINE>(a, keys, s); break;
        default: launch_ref_rescore_op<FMT, OP_L2>(a, keys, s); break;
    }
}

hipError_t launch_ref_rescore(const RefArgs& a, uint64_t* keys, hipStream_t s) {
    if (a.d <= 0 || a.d > kMaxQueryDim || a.kp <= 0 || a.nq <= 0 || a.nq > 65535) return hipErrorInvalidValue;
    if (a.fmt == 4 && a.d % 32 != 0) return hipErrorInvalidValue;
    if (a.fmt == 8) launch_ref_rescore_fmt<8>(a, keys, s);
    else launch_ref_rescore_fmt<4>(a, keys, s);
    return hipGetLastError();
}

hipError_t launch_ref_finish(const RefArgs& a, const uint64_t* keys, hipStream_t s) {
    if (a.d <= 0 || a.d > kMaxQueryDim || a.k <= 0 || a.kp < a.k || a.nq <= 0) return hipErrorInvalidValue;
    const int S = next_pow2_host(a.kp);
    if (S > kRefMaxKeys) return hipErrorInvalidValue;
    const size_t lds = (size_t)S * 8;
    const dim3 grid((unsigned)a.nq);
    // 1024 threads sort the larger candidate sets (fewer register slots and
    // network steps per thread)
    if (S > 512) {
        switch (a.op) {
            case OP_DOT: hipLaunchKernelGGL((ref_finish_kernel<OP_DOT, 1024>), grid, dim3(1024), lds, s, a, keys); break;
            case OP_COSINE:
                hipLaunchKernelGGL((ref_finish_kernel<OP_COSINE, 1024>), grid, dim3(1024), lds, s, a, keys);
                break;
            default: hipLaunchKernelGGL((ref_finish_kernel<OP_L2, 1024>), grid, dim3(1024), lds, s, a, keys); break;
        }
    } else {
        switch (a.op) {
            case OP_DOT: hipLaunchKernelGGL((ref_finish_kernel<OP_DOT, 256>), grid, dim3(256), lds, s, a, keys); break;
            case OP_COSINE:
                hipLaunchKernelGGL((ref_finish_kernel<OP_COSINE, 256>), grid, dim3(256), lds, s, a, keys);
                break;
            default: hipLaunchKernelGGL((ref_finish_kernel<OP_L2, 256>), grid, dim3(256), lds, s, a, keys); break;
        }
    }
    return hipGetLastError();
}

template <int FMT>
static hipError_t launch_ref_scan_fmt(int op, const ScanArgs& a, int nq, const double* sqd, const int* redo,
                                      const uint64_t* redo_tau, dim3 grid, size_t lds, hipStream_t s) {
    const dim3 block(256);
    switch (op) {
        case OP_DOT:
            hipLaunchKernelGGL((ref_scan_kernel<FMT, OP_DOT>), grid, block, lds, s, a, nq, sqd, redo, redo_tau);
            break;
        case OP_COSINE:
            hipLaunchKernelGGL((ref_scan_kernel<FMT, OP_COSINE>), grid, block, lds, s, a, nq, sqd, redo, redo_tau);
            break;
        default:
            hipLaunchKernelGGL((ref_scan_kernel<FMT, OP_L2>), grid, block, lds, s, a, nq, sqd, redo, redo_tau);
            break;
    }
    return hipGetLastError();
}

hipError_t launch_ref_scan(int fmt, int op, const ScanArgs& a, int nq, const double* sqd, const int* redo,
                           const uint64_t* redo_tau, dim3 grid, size_t lds, hipStream_t s) {
    if (a.d <= 0 || a.d > kMaxQueryDim || nq <= 0) return hipErrorInvalidValue;
    if (fmt == 4 && a.d % 32 != 0) return hipErrorInvalidValue;
    return fmt == 8 ? launch_ref_scan_fmt<8>(op, a, nq, sqd, redo, redo_tau, grid, lds, s)
                    : launch_ref_scan_fmt<4>(op, a, nq, sqd, redo, redo_tau, grid, lds, s);
}

}  // namespace manta
