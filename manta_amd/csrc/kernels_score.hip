// kernels_score.hip -- packed-candidate scoring for gfx950 (streaming path).
//
// One launch per fused score+top-k call.  Each workgroup (256 threads, 4
// waves) encodes its query into LDS, then scores `rounds` x 256 candidate
// rows against it.  q8 rows are read with coalesced 16-byte loads: L lanes
// cover one row (L*16 contiguous bytes per load), C loads per lane per row,
// so a wave moves 64*16 bytes per load instruction.  The int8 products run
// on v_dot4 with the query codes held in registers; row sums are reduced
// across the L lanes with xor shuffles and then transposed so that thread t
// owns row t of the round.  The epilogue computes the exact f32 score of the
// packed contract and either stores it (score matrix) or feeds the LDS top-k
// reservoir.  In top-k mode each workgroup writes its k best keys; the last
// workgroup of a query (atomic ticket) merges them into the final ids.
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

// E8 (q8 dot): qmax = max(1, maxabs), code = clamp(round((q*127)/qmax)).
__device__ __forceinline__ int code_e8(float x, float qmax) {
    float r = round_half_away(fdiv_rn(fmul_rn(x, 127.0f), qmax));
    return (int)fminf(127.0f, fmaxf(-127.0f, r));
}

// E16: code = clamp(round(q*(32639/maxabs)), +-32639), split 256*hi + lo
// with lo the signed low byte.
__device__ __forceinline__ int code_e16(float x, float inv) {
    float r = round_half_away(fmul_rn(x, inv));
    return (int)fminf(32639.0f, fmaxf(-32639.0f, r));
}

__device__ __forceinline__ QConst e16_consts(float maxabs, long long ss) {
    QConst k{0.0f, 0.0f, 0.0f, 0.0f};
    if (maxabs != 0.0f) {
        const float qs = fdiv_rn(maxabs, 32639.0f);
        const double dss = (double)ss;
        k.a = qs;
        k.b = (float)__dmul_rn(__dsqrt_rn(dss), (double)qs);
        k.c = (float)__dmul_rn(__dmul_rn(dss, (double)qs), (double)qs);
    }
    return k;
}

// q4 digit planes are permuted per 8 columns to [c0 c2 c4 c6 c1 c3 c5 c7]
// so that the nibble unpack below feeds v_dot4 without shuffling.
__device__ __forceinline__ int q4_perm_pos(int c) {
    const int j = c & 7;
    return (c & ~7) + ((j & 1) ? 4 + (j >> 1) : (j >> 1));
}

enum { ENC_E8 = 0, ENC_E16 = 1, ENC_E16_Q4 = 2 };

struct QueryLds {
    int8_t c8[kMaxQueryDim];
    int8_t hi[kMaxQueryDim];
    int8_t lo[kMaxQueryDim];
    QConst qc;
    float redf[4];
    long long redi[4];
};

// Encode one f16 query into LDS (whole workgroup, 256 threads).  `span` is
// the number of code slots to fill (the row pitch; columns >= d get 0).
__device__ inline void encode_query_block(const uint16_t* __restrict__ qrow, int d, int span, int enc,
                                          QueryLds& L) {
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    float m = 0.0f;
    for (int c = tid; c < d; c += 256) m = fmaxf(m, __builtin_fabsf(h2f(qrow[c])));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (lane == 0) L.redf[wave] = m;
    __syncthreads();
    const float maxabs = fmaxf(fmaxf(L.redf[0], L.redf[1]), fmaxf(L.redf[2], L.redf[3]));
    if (enc == ENC_E8) {
        const float qmax = fmaxf(1.0f, maxabs);
        for (int c = tid; c < span; c += 256) L.c8[c] = (int8_t)(c < d ? code_e8(h2f(qrow[c]), qmax) : 0);
        if (tid == 0) L.qc = QConst{qmax, 0.0f, 0.0f, 0.0f};
        __syncthreads();
        return;
    }
    const float inv = maxabs == 0.0f ? 0.0f : fdiv_rn(32639.0f, maxabs);
    long long ss = 0;
    for (int c = tid; c < span; c += 256) {
        const int code = (c < d && maxabs != 0.0f) ? code_e16(h2f(qrow[c]), inv) : 0;
        const int l = (int)(int8_t)(code & 0xFF);
        const int h = (code - l) >> 8;
        const int pos = enc == ENC_E16_Q4 ? q4_perm_pos(c) : c;
        L.hi[pos] = (int8_t)h;
        L.lo[pos] = (int8_t)l;
        ss += (long long)code * code;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    if (lane == 0) L.redi[wave] = ss;
    __syncthreads();
    if (tid == 0) L.qc = e16_consts(maxabs, L.redi[0] + L.redi[1] + L.redi[2] + L.redi[3]);
    __syncthreads();
}

// Global-memory variant: one workgroup per query (used by the batched
// paths, whose many workgroups share each query).
__global__ __launch_bounds__(256) void query_encode_kernel(const uint16_t* __restrict__ q, int d, int pitch,
                                                           int e16, int8_t* __restrict__ c8,
                                                           int8_t* __restrict__ hi, int8_t* __restrict__ lo,
                                                           QConst* __restrict__ qc) {
    __shared__ QueryLds L;
    const int qi = blockIdx.x;
    // e16: 0 = E8 codes, 1 = E16 digit planes, 2 = E16 planes in the q4 nibble order
    encode_query_block(q + (int64_t)qi * d, d, pitch, e16 == 2 ? ENC_E16_Q4 : (e16 ? ENC_E16 : ENC_E8), L);
    for (int c = threadIdx.x; c < pitch; c += 256) {
        if (e16) {
            hi[(int64_t)qi * pitch + c] = L.hi[c];
            lo[(int64_t)qi * pitch + c] = L.lo[c];
        } else {
            c8[(int64_t)qi * pitch + c] = L.c8[c];
        }
    }
    if (threadIdx.x == 0) qc[qi] = L.qc;
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

// ------------------------------------------------------- top-k plumbing

struct ScanLds {
    QueryLds q;
    TopKShared st;
    int last;
};

// Store the score, or offer it to the reservoir.
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

// End of a top-k scan workgroup: publish its k best keys; the last
// workgroup of the query (ticket == gridDim.x - 1) merges every part into
// the final sorted ids / scores and resets the ticket for the next call.
// Publication avoids device-wide fences (each one writes back and
// invalidates a whole XCD L2): the keys are stored write-through at agent
// scope (sc1), every thread waits for its stores to complete before the
// barrier, the ticket is an agent-scope atomic, and the merging workgroup
// reads the parts with agent-scope (sc1) loads.
__device__ inline void finish_topk(const ScanArgs& a, uint64_t* keys, ScanLds& S, int qi) {
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

// -------------------------------------------------- q8, coalesced lanes

template <int OP, int L, int C>
__global__ __launch_bounds__(256) void q8_scan_kernel(ScanArgs a) {
    extern __shared__ uint64_t topk_keys[];
    __shared__ ScanLds S;
    constexpr int G = 64 / L;  // rows per wave per load step
    const int qi = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int p = lane % L;
    const int g = lane / L;
    const int64_t set_row0 = (int64_t)qi * a.set_stride;
    const int8_t* __restrict__ codes = a.codes + set_row0 * a.pitch;
    const float* __restrict__ scales = (const float*)a.scales + set_row0;

    encode_query_block(a.queries + (int64_t)qi * a.d, a.d, a.pitch, OP == OP_DOT ? ENC_E8 : ENC_E16, S.q);
    const QConst kq = S.q.qc;
    v4i qa[C], qb[C];
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int off = c * 16 * L + p * 16;
        if (OP == OP_DOT) {
            qa[c] = *(const v4i*)(S.q.c8 + off);
            qb[c] = qa[c];
        } else {
            qa[c] = *(const v4i*)(S.q.hi + off);
            qb[c] = *(const v4i*)(S.q.lo + off);
        }
    }
    if (!a.out_scores) topk_init(topk_keys, &S.st);

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
        const uint64_t tau = a.out_scores ? 0ull : S.st.tau;
        emit_round(score, valid, row, a.n, qi, a.out_scores, topk_keys, &S.st, tau, a.smallest);
        if (!a.out_scores && a.mid_compact) {
            __syncthreads();
            topk_maybe_compact(topk_keys, &S.st, a.k, a.cap);
        }
    }
    if (!a.out_scores) finish_topk(a, topk_keys, S, qi);
}

// --------------------------------------------- q8, any pitch (lane = row)

template <int OP>
__global__ __launch_bounds__(256) void q8_scan_generic_kernel(ScanArgs a) {
    extern __shared__ uint64_t topk_keys[];
    __shared__ ScanLds S;
    const int qi = blockIdx.y;
    const int64_t set_row0 = (int64_t)qi * a.set_stride;
    const int8_t* __restrict__ codes = a.codes + set_row0 * a.pitch;
    const float* __restrict__ scales = (const float*)a.scales + set_row0;
    encode_query_block(a.queries + (int64_t)qi * a.d, a.d, a.pitch, OP == OP_DOT ? ENC_E8 : ENC_E16, S.q);
    const QConst kq = S.q.qc;
    const int8_t* qa = OP == OP_DOT ? S.q.c8 : S.q.hi;
    const int8_t* qb = S.q.lo;
    const int chunks = a.pitch / 16;
    if (!a.out_scores) topk_init(topk_keys, &S.st);
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
        const uint64_t tau = a.out_scores ? 0ull : S.st.tau;
        emit_round(score, valid, row, a.n, qi, a.out_scores, topk_keys, &S.st, tau, a.smallest);
        if (!a.out_scores && a.mid_compact) {
            __syncthreads();
            topk_maybe_compact(topk_keys, &S.st, a.k, a.cap);
        }
    }
    if (!a.out_scores) finish_topk(a, topk_keys, S, qi);
}

// ------------------------------------------------------- q4 (lane = row)

// Nibbles to 16x-scaled int8 lanes: (w << 4) & 0xF0F0F0F0 holds the even
// nibbles of w as 16*code, w & 0xF0F0F0F0 the odd ones; the query digit
// planes are permuted to match (q4_perm_pos).  Block sums are 16x the true
// sums and are divided back exactly.
template <int OP>
__global__ __launch_bounds__(256) void q4_scan_kernel(ScanArgs a) {
    extern __shared__ uint64_t topk_keys[];
    __shared__ ScanLds S;
    const int qi = blockIdx.y;
    const int64_t set_row0 = (int64_t)qi * a.set_stride;
    const uint8_t* __restrict__ packed = (const uint8_t*)a.codes + set_row0 * a.pitch;
    const uint16_t* __restrict__ scales = (const uint16_t*)a.scales + set_row0 * a.nb;
    encode_query_block(a.queries + (int64_t)qi * a.d, a.d, a.d, ENC_E16_Q4, S.q);
    const QConst kq = S.q.qc;
    const int* qh = (const int*)S.q.hi;
    const int* ql = (const int*)S.q.lo;
    if (!a.out_scores) topk_init(topk_keys, &S.st);
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
        const uint64_t tau = a.out_scores ? 0ull : S.st.tau;
        emit_round(score, valid, row, a.n, qi, a.out_scores, topk_keys, &S.st, tau, a.smallest);
        if (!a.out_scores && a.mid_compact) {
            __syncthreads();
            topk_maybe_compact(topk_keys, &S.st, a.k, a.cap);
        }
    }
    if (!a.out_scores) finish_topk(a, topk_keys, S, qi);
}

// ------------------------------------------------ exact accumulator rescore

// One workgroup per query: re-encode the query and recompute the q8
// integer accumulator of each selected row (E8 for dot, E16 hi/lo combined
// for the others), written as int64.
__global__ __launch_bounds__(256) void q8_rescore_acc_kernel(const int8_t* __restrict__ codes, int pitch,
                                                             int64_t set_stride, int64_t n, int d,
                                                             const uint16_t* __restrict__ queries,
                                                             const int32_t* __restrict__ ids, int k, int e16,
                                                             int64_t* __restrict__ out) {
    __shared__ QueryLds L;
    const int qi = blockIdx.x;
    encode_query_block(queries + (int64_t)qi * d, d, pitch, e16 ? ENC_E16 : ENC_E8, L);
    for (int i = threadIdx.x; i < k; i += blockDim.x) {
        const int64_t row = ids[(int64_t)qi * k + i];
        int64_t acc = 0;
        if (row >= 0 && row < n) {
            const int8_t* rp = codes + ((int64_t)qi * set_stride + row) * pitch;
            for (int c = 0; c < pitch; c++)
                acc += (int64_t)rp[c] * (e16 ? 256 * (int64_t)L.hi[c] + L.lo[c] : (int64_t)L.c8[c]);
        }
        out[(int64_t)qi * k + i] = acc;
    }
}

// ----------------------------------------------------------------- hosts

hipError_t launch_query_encode(const uint16_t* q, int nq, int d, int pitch, int e16, int8_t* c8,
                               int8_t* hi, int8_t* lo, QConst* qc, hipStream_t s) {
    hipLaunchKernelGGL(query_encode_kernel, dim3(nq), dim3(256), 0, s, q, d, pitch, e16, c8, hi, lo, qc);
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

hipError_t launch_q8_rescore(const int8_t* codes, int pitch, int64_t set_stride, int64_t n, int d,
                             const uint16_t* queries, const int32_t* ids, int k, int nq, int e16,
                             int64_t* out, hipStream_t s) {
    hipLaunchKernelGGL(q8_rescore_acc_kernel, dim3(nq), dim3(256), 0, s, codes, pitch, set_stride, n, d,
                       queries, ids, k, e16, out);
    return hipGetLastError();
}

}  // namespace manta
