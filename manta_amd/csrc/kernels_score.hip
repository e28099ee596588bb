// kernels_score.hip -- packed-candidate scoring for gfx950 (streaming path).
//
// One launch per fused score+top-k call.  Each workgroup (256 threads, 4
// waves) scores `rounds` x 256 candidate rows against one query.  q8 rows
// are read with coalesced 16-byte buffer loads: L lanes cover one row (L*16
// contiguous bytes per load), C loads per lane per row, so a wave moves
// 64*16 bytes per load instruction.  The int8 products run on v_dot4 with
// the query codes held in registers (each lane encodes the columns it
// multiplies); a DPP group sum over the L lanes leaves every lane of a group
// the row total, and lane g*L + j keeps row g*L + j, so after a round each
// lane owns one row for the epilogue.  The epilogue computes the f32 score
// and either stores it (score matrix) or offers its key to per-wave sorted
// register lists (k <= 64) or the LDS reservoir.  In top-k mode each
// workgroup publishes its k best keys; the last workgroup of a query (atomic
// ticket) merges them into the final ids.
//
// Quantized-query scores (the CPU oracle restates them):
//   q8 dot    (E8 query codes):  t = s_r*acc; t = t*qmax; score = t/127
//             (BASELINE's q8 dot formula, the quantized-query dot);
//   q8 E16 codes (hi/lo digits): qd = (s_r*qs)*f32(acc); dot16 = qd;
//             cosine = den == 0 ? 0 : qd/den with den = |q|*|d_r|;
//             l2 = sqrt(max(0, (qq + dd_r) - 2*qd));
//   q4        (E16):             qd = qs * fma-chain over blocks of
//                                f16scale_b * f32(acc_b); then as above.
// The E16 scores rank rows for the reference-semantics top-k, which
// rescores the best of them with the reference's arithmetic
// (kernels_ref.hip).
#include "device_common.hpp"
#include "kernels.hpp"
#include "q4_common.hpp"
#include "scan_common.hpp"

namespace manta {

// ------------------------------------------------------------ query codes

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
                                                           QConst* __restrict__ qc, uint64_t* __restrict__ tau,
                                                           int* __restrict__ bcnt) {
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
    if (threadIdx.x == 0) {
        qc[qi] = L.qc;
        // the threshold passes start from no threshold and no kept keys
        if (tau) tau[qi] = 0ull;
        if (bcnt) bcnt[qi] = 0;
    }
}

// Shadow-scan query encoding (one workgroup per query): the E16 planes in
// the q4 order and constants as above, full-range int8 codes
// c = round(q * 127/maxabs) with qa = maxabs/127 for the shadow's A operand,
// and shadow_bound's margin m and factor f.  With q^ the E16-dequantized
// query and G = |q^ - qa c|, a row's exact score and its shadow pre-score
// p differ by at most E/|x| + (F/|x|) G/|q^| (cosine, in score units; p
// scaled by f = |q^|/qa) or E|q^| + F G (dot, f = 1/qa), E and F the
// shadow's row error terms (ShadowInfo maxima); m adds 2^-16 (times the
// largest |x||q^| for dot), far above every f32 rounding on either side.
__global__ __launch_bounds__(256) void query_encode_shadow_kernel(const uint16_t* __restrict__ q, int d, int spitch,
                                                                  int op, const ShadowInfo* __restrict__ info,
                                                                  int8_t* __restrict__ c8, int8_t* __restrict__ hi,
                                                                  int8_t* __restrict__ lo, QConst* __restrict__ qc,
                                                                  float* __restrict__ qb, uint64_t* __restrict__ tau,
                                                                  int* __restrict__ bcnt) {
    __shared__ QueryLds L;
    __shared__ double g2s[4];
    __shared__ long long sss[4];
    const int qi = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const uint16_t* qrow = q + (int64_t)qi * d;
    encode_query_block(qrow, d, d, ENC_E16_Q4, L);
    const float maxabs = fmaxf(fmaxf(L.redf[0], L.redf[1]), fmaxf(L.redf[2], L.redf[3]));
    const float qs = L.qc.a;
    const float inv16 = maxabs == 0.0f ? 0.0f : fdiv_rn(32639.0f, maxabs);
    const float qa = fdiv_rn(maxabs, 127.0f);
    const float inv8 = maxabs == 0.0f ? 0.0f : fdiv_rn(127.0f, maxabs);
    double g2 = 0.0;
    long long ss = 0;
    for (int c = tid; c < spitch; c += 256) {
        int k8 = 0;
        if (c < d && maxabs != 0.0f) {
            const float x = h2f(qrow[c]);
            k8 = (int)fminf(127.0f, fmaxf(-127.0f, round_half_away(fmul_rn(x, inv8))));
            const int k16 = code_e16(x, inv16);
            const double diff = (double)k16 * (double)qs - (double)k8 * (double)qa;
            g2 += diff * diff;
            ss += (long long)k16 * k16;
        }
        c8[(int64_t)qi * spitch + c] = (int8_t)k8;
    }
    for (int c = tid; c < d; c += 256) {
        hi[(int64_t)qi * d + c] = L.hi[c];
        lo[(int64_t)qi * d + c] = L.lo[c];
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        g2 += __shfl_xor(g2, off);
        ss += __shfl_xor(ss, off);
    }
    if (lane == 0) {
        g2s[wave] = g2;
        sss[wave] = ss;
    }
    __syncthreads();
    if (tid == 0) {
        qc[qi] = L.qc;
        if (tau) tau[qi] = 0ull;
        if (bcnt) bcnt[qi] = 0;
        const double G = __builtin_sqrt(g2s[0] + g2s[1] + g2s[2] + g2s[3]);
        const double qn = __builtin_sqrt((double)(sss[0] + sss[1] + sss[2] + sss[3])) * (double)qs;
        const double up = 1.0 + 9.5367431640625e-7;
        float m = 0.0f, f = 0.0f;
        if (qn > 0.0) {
            const double me_c = __uint_as_float(info->me_cos), mf_c = __uint_as_float(info->mf_cos);
            const double me_d = __uint_as_float(info->me_dot), mf_d = __uint_as_float(info->mf_dot);
            const double mn = __uint_as_float(info->maxn);
            if (op == OP_COSINE) {
                m = (float)((me_c + mf_c * G / qn + 1.52587890625e-05) * up);
                f = (float)(qn / (double)qa);
            } else {
                m = (float)((me_d * qn + mf_d * G + 1.52587890625e-05 * mn * qn) * up);
                f = (float)(1.0 / (double)qa);
            }
        }
        qb[2 * qi] = m;
        qb[2 * qi + 1] = f;
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
    if (OP == OP_DOT16) return qd;
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

// End of a top-k scan workgroup on the wave-list path (k <= 64): the waves'
// lists merge into wave 0's, which publishes the workgroup's k best keys
// (sorted) as finish_topk does; the last workgroup of the query merges all
// parts with the same lists, 8 keys per lane in flight, and writes ids and
// scores straight from wave 0's lanes.  buf: blockDim.x keys of LDS.
template <class SL>
__device__ inline void finish_wave_lists(const ScanArgs& a, uint64_t list, uint64_t thr, uint64_t* buf, SL& S,
                                         int qi) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    wave_lists_merge(list, thr, a.k, buf);
    const int64_t per_q = (int64_t)gridDim.x * a.k;
    uint64_t* dst = a.partial + (int64_t)qi * per_q + (int64_t)blockIdx.x * a.k;
    if (wave == 0 && lane < a.k) __hip_atomic_store(dst + lane, list, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Publication order at the ISA level (gfx950): every access to the parts
    // and the ticket is an agent-scope atomic, which the AMDGPU memory model
    // implements as sc1 accesses performed at the device coherence point
    // (past the per-XCD L2s); s_waitcnt vmcnt(0) retires this wave's part
    // stores there before the barrier, the ticket RMW is issued after it,
    // and the last workgroup's sc1 loads read the coherence point.  A
    // source-level release/acquire pair would add an L2 writeback per
    // workgroup (buffer_wbl2): 11% more time on a 32-problem q8 scan.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        S.last = __hip_atomic_fetch_add(&a.tickets[qi], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 gridDim.x - 1;
    __syncthreads();
    if (!S.last) return;
    const uint64_t* src = a.partial + (int64_t)qi * per_q;
    // Up to one part key per thread (C0's 32-problem launch: 8 parts of 10):
    // every key counts the keys above it and the k best land at their ranks,
    // no insertions on the launch's last step.
    if (per_q <= (int64_t)blockDim.x) {
        __shared__ uint64_t res[64];  // k <= 64 on the list path
        const int t = (int)threadIdx.x, n = (int)per_q, k = a.k;
        const uint64_t mine = t < n ? __hip_atomic_load(src + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
        buf[t] = mine;
        if (t < 64) res[t] = 0ull;
        __syncthreads();
        int rank = 0;
        if (mine)
            for (int i = 0; i < n; i++) rank += buf[i] > mine ? 1 : 0;
        if (mine && rank < k) res[rank] = mine;  // keys are distinct: so are their ranks
        __syncthreads();
        if (t < k) {
            const uint64_t key = res[t];
            a.out_ids[(int64_t)qi * k + t] = key ? (int32_t)key_index(key) : -1;
            if (a.out_topk_scores) a.out_topk_scores[(int64_t)qi * k + t] = key ? key_score(key, a.smallest) : 0.0f;
        }
        if (t == 0) __hip_atomic_store(&a.tickets[qi], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    // Many parts (a single query's call: 128 parts of k): the k-th largest
    // part head is a floor of the final k-th key (the k best heads are k
    // distinct keys), only the k parts whose heads reach it hold keys at or
    // above it, and those k^2 or fewer candidates take their place by rank
    // (each counts the candidates above it) instead of one insertion each.
    // Fewer than k keys in the parts' heads: the lists below.
    if (a.k <= 16 && (int)gridDim.x >= a.k && gridDim.x <= 256) {
        __shared__ uint64_t heads[256];
        __shared__ uint64_t floor_s;
        __shared__ int ncand;
        const int t = (int)threadIdx.x, P = (int)gridDim.x, k = a.k;
        uint64_t mk[16];
#pragma unroll
        for (int j = 0; j < 16; j++)
            mk[j] = (t < P && j < k) ? __hip_atomic_load(src + (int64_t)t * k + j, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT)
                                     : 0ull;
        heads[t] = mk[0];  // a part's list is sorted: its first key is its best
        if (t == 0) {
            floor_s = 0ull;
            ncand = 0;
        }
        __syncthreads();
        if (t < P && mk[0]) {
            int rank = 0;
            for (int i = 0; i < P; i++) rank += heads[i] > mk[0] ? 1 : 0;
            if (rank == k - 1) floor_s = mk[0];  // keys are distinct: one thread
        }
        __syncthreads();
        const uint64_t fl = floor_s;
        if (fl) {
            int cnt = 0;
#pragma unroll
            for (int j = 0; j < 16; j++) cnt += mk[j] >= fl ? 1 : 0;  // (empty slots are 0 < fl)
            if (t < P && cnt) {
                int pos = atomicAdd(&ncand, cnt);
#pragma unroll
                for (int j = 0; j < 16; j++)
                    if (mk[j] >= fl) buf[pos++] = mk[j];
            }
            __syncthreads();
            const int nc = ncand;  // k <= nc <= k^2 <= blockDim.x
            const uint64_t mine = t < nc ? buf[t] : 0ull;
            int rank = 0;
            if (t < nc)
                for (int i = 0; i < nc; i++) rank += buf[i] > mine ? 1 : 0;
            __syncthreads();  // every read of buf is done
            if (t < nc && rank < k) buf[rank] = mine;
            __syncthreads();
            if (t < k) {
                const uint64_t key = buf[t];
                a.out_ids[(int64_t)qi * k + t] = (int32_t)key_index(key);
                if (a.out_topk_scores) a.out_topk_scores[(int64_t)qi * k + t] = key_score(key, a.smallest);
            }
            if (t == 0) __hip_atomic_store(&a.tickets[qi], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
    }
    list = 0;
    thr = 0;
    // batches of 64 keys go to the waves in turn; B batches per wave in flight
    constexpr int B = 8;
    const int64_t stride = (int64_t)blockDim.x;
    for (int64_t base = (int64_t)wave * 64; base < per_q; base += stride * B) {
        uint64_t kb[B];
#pragma unroll
        for (int b = 0; b < B; b++) {
            const int64_t i = base + b * stride + lane;
            kb[b] = i < per_q ? __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
        }
#pragma unroll
        for (int b = 0; b < B; b++) wave_list_offer(kb[b], list, thr, a.k);
    }
    wave_lists_merge(list, thr, a.k, buf);
    if (wave == 0 && lane < a.k) {
        a.out_ids[(int64_t)qi * a.k + lane] = list ? (int32_t)key_index(list) : -1;
        if (a.out_topk_scores) a.out_topk_scores[(int64_t)qi * a.k + lane] = list ? key_score(list, a.smallest) : 0.0f;
    }
    if (threadIdx.x == 0) __hip_atomic_store(&a.tickets[qi], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// -------------------------------------------------- q8, coalesced lanes

// Sum over aligned groups of L lanes (L = 4, 8 or 16) with DPP moves inside
// each 16-lane row; every lane of a group receives the group total.
template <int L>
__device__ __forceinline__ int group_sum(int s) {
    s += __builtin_amdgcn_update_dpp(0, s, 0xB1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
    s += __builtin_amdgcn_update_dpp(0, s, 0x4E, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
    if (L >= 8) s += __builtin_amdgcn_update_dpp(0, s, 0x141, 0xf, 0xf, false);   // row_half_mirror
    if (L >= 16) s += __builtin_amdgcn_update_dpp(0, s, 0x140, 0xf, 0xf, false);  // row_mirror
    return s;
}

// Buffer resource over `bytes` bytes at p (raw, stride 0): loads at offsets
// at or past `bytes` return zero instead of touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t byte_buffer(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// DPP move of a double: both 32-bit halves with the same pattern.
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double x) {
    const uint64_t b = __builtin_bit_cast(uint64_t, x);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xf, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xf, 0xf, false);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

template <int L>
__device__ __forceinline__ float group_fmax(float m) {
    m = fmaxf(m, dpp_f32<0xB1>(m));
    m = fmaxf(m, dpp_f32<0x4E>(m));
    if (L >= 8) m = fmaxf(m, dpp_f32<0x141>(m));
    if (L >= 16) m = fmaxf(m, dpp_f32<0x140>(m));
    return m;
}

// Exact while every partial sum stays below 2^53 (sums of squared codes).
template <int L>
__device__ __forceinline__ double group_dsum(double s) {
    s += dpp_f64<0xB1>(s);
    s += dpp_f64<0x4E>(s);
    if (L >= 8) s += dpp_f64<0x141>(s);
    if (L >= 16) s += dpp_f64<0x140>(s);
    return s;
}

// Encode the query columns this lane multiplies straight into registers:
// chunk c of lane p covers columns [16*(c*L + p), +16) (zero past d).  The L
// lanes of a group cover every column, so group reductions give the
// whole-query max |q| and sum of squared codes; codes and constants equal
// encode_query_block's.  Whole wave, no LDS, no barrier.
template <int OP, int L, int C>
__device__ __forceinline__ QConst encode_query_lanes(const uint16_t* qrow, int d, int p, v4i* qa, v4i* qb) {
    const __amdgpu_buffer_rsrc_t qr = byte_buffer(qrow, (uint32_t)d * 2u);
    uint16_t hx[C][16];  // raw f16 bits, converted where used
    float m = 0.0f;
#pragma unroll
    for (int c = 0; c < C; c++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int col = c * 16 * L + p * 16 + e;
            hx[c][e] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(qr, col * 2, 0, 0);
            m = fmaxf(m, __builtin_fabsf(h2f(hx[c][e])));
        }
    m = group_fmax<L>(m);
    if (OP == OP_DOT) {
        const float qmax = fmaxf(1.0f, m);
#pragma unroll
        for (int c = 0; c < C; c++) {
#pragma unroll
            for (int w = 0; w < 4; w++) {
                int word = 0;
#pragma unroll
                for (int b = 0; b < 4; b++) word |= (code_e8(h2f(hx[c][4 * w + b]), qmax) & 0xFF) << (8 * b);
                qa[c][w] = word;
            }
            qb[c] = qa[c];
        }
        return QConst{qmax, 0.0f, 0.0f, 0.0f};
    }
    const float inv = m == 0.0f ? 0.0f : fdiv_rn(32639.0f, m);
    double ss = 0.0;
#pragma unroll
    for (int c = 0; c < C; c++)
#pragma unroll
        for (int w = 0; w < 4; w++) {
            int hw = 0, lw = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int code = m != 0.0f ? code_e16(h2f(hx[c][4 * w + b]), inv) : 0;
                const int l = (int)(int8_t)(code & 0xFF);
                const int h = (code - l) >> 8;
                hw |= (h & 0xFF) << (8 * b);
                lw |= (l & 0xFF) << (8 * b);
                ss += (double)code * (double)code;
            }
            qa[c][w] = hw;
            qb[c][w] = lw;
        }
    ss = group_dsum<L>(ss);
    return e16_consts(m, (long long)ss);
}

// Pitch = 16*L*C bytes.  A wave scores a block of 64 rows per round; lane
// group g (L lanes) owns rows g*L .. g*L+L-1 of the block.  Load (j, c)
// reads row g*L + j, lane p of the group taking bytes [16p + 16Lc, +16), so
// one load instruction reads 64/L whole rows.  The row sum is a DPP group
// sum, and lane g*L + j keeps it: after a round every lane holds the
// accumulator of its own row.  Loads go through a buffer resource clipped to
// the workgroup's rows (no branch per load; rows past n read zero and are
// masked by `valid`).
template <int OP, int L, int C, bool LISTS>
__global__ __launch_bounds__(256) void q8_scan_kernel(ScanArgs a) {
    extern __shared__ uint64_t topk_keys[];
    __shared__ ScanTopkLds S;
    __shared__ uint64_t ff_keys[LISTS ? 256 : 1];  // the lists' first fill, 64 keys a wave
    constexpr int PITCH = 16 * L * C;
    constexpr int JS0 = C == 1 ? 16 : (C == 2 ? 8 : 4);  // rows per load step (<= 16 loads)
    constexpr int JS = JS0 < L ? JS0 : L;
    static_assert(L % JS == 0, "load steps must tile the lane group");
    const int qi = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int p = lane % L;
    const int g = lane / L;
    const int64_t set_row0 = (int64_t)qi * a.set_stride;
    const int8_t* __restrict__ codes = a.codes + set_row0 * PITCH;
    const float* __restrict__ scales = (const float*)a.scales + set_row0;

    const int64_t wg_row0 = (int64_t)blockIdx.x * a.rounds * 256;
    const int64_t left = a.n - wg_row0;  // > 0: the grid covers n exactly
    const int wg_rows = left < (int64_t)a.rounds * 256 ? (int)left : a.rounds * 256;
    const __amdgpu_buffer_rsrc_t rs = byte_buffer(codes + wg_row0 * PITCH, (uint32_t)wg_rows * PITCH);
    const int lane_off = g * L * PITCH + p * 16;
    // One load step: rows j0 .. j0+JS-1 of every lane group of the wave's
    // block in round r.  On the wave-list path the next step's loads are
    // issued as soon as the current step's values are consumed, so they
    // overlap the epilogue and the top-k offer, and the first step's overlap
    // the query encoding.
    v4i v[JS][C];
    auto load_step = [&](int r, int j0) {
        const int vb = (r * 256 + wave * 64) * PITCH + lane_off;
#pragma unroll
        for (int j = 0; j < JS; j++)
#pragma unroll
            for (int c = 0; c < C; c++)
                v[j][c] = __builtin_amdgcn_raw_buffer_load_b128(rs, vb + (j0 + j) * PITCH + c * 16 * L, 0, 2);
    };
    if (LISTS) load_step(0, 0);

    v4i qa[C], qb[C];
    const QConst kq = encode_query_lanes<OP, L, C>(a.queries + (int64_t)qi * a.d, a.d, p, qa, qb);
    // LISTS: top-k through per-wave register lists (k <= 64, never score mode)
    uint64_t list = 0, thr = 0;
    if (!LISTS && !a.out_scores) topk_init(topk_keys, &S.st);

    for (int r = 0; r < a.rounds; r++) {
        const int64_t row = wg_row0 + r * 256 + wave * 64 + lane;
        const bool valid = row < a.n;
        const int64_t crow = valid ? row : a.n - 1;
        const float sc = scales[crow];
        float dn = 0.0f, d2 = 0.0f;
        if (OP == OP_COSINE) dn = a.dnorm[set_row0 + crow];
        if (OP == OP_L2) d2 = a.dd[set_row0 + crow];
        int my_hi = 0, my_lo = 0;
#pragma unroll
        for (int j0 = 0; j0 < L; j0 += JS) {
            // the reservoir path loads each step when it starts (its offer
            // and compaction would otherwise run with a step of loads held)
            if (!LISTS) load_step(r, j0);
#pragma unroll
            for (int j = 0; j < JS; j++) {
                int s_hi = 0, s_lo = 0;
#pragma unroll
                for (int c = 0; c < C; c++) {
                    s_hi = dot16(v[j][c], qa[c], s_hi);
                    if (OP != OP_DOT) s_lo = dot16(v[j][c], qb[c], s_lo);
                }
                s_hi = group_sum<L>(s_hi);
                if (OP != OP_DOT) s_lo = group_sum<L>(s_lo);
                if (p == j0 + j) {
                    my_hi = s_hi;
                    my_lo = s_lo;
                }
            }
            // the step's values are consumed before the next loads are
            // issued (else the loads would be hoisted and double the
            // registers held)
            asm volatile("" : "+v"(my_hi), "+v"(my_lo));
            asm volatile("" ::: "memory");
            if (!LISTS) continue;
            // unconditional, so the wait counts stay static: after the last
            // round these loads fall past the buffer and return zeros
            // without touching memory
            if (j0 + JS < L)
                load_step(r, j0 + JS);
            else
                load_step(r + 1, 0);
        }
        float score = 0.0f;
        if (valid) score = q8_epilogue<OP>(my_hi, my_lo, sc, kq, dn, d2);
        if (LISTS) {
            const uint64_t key = valid ? make_key(score, (uint32_t)row, a.smallest) : 0ull;
            // (the lists start empty: the first round fills them by rank,
            // in LDS of its own -- a wave that finishes early may already be
            // merging through topk_keys)
            if (r == 0) wave_list_first_fill(key, list, thr, a.k, ff_keys + wave * 64);
            else wave_list_offer(key, list, thr, a.k);
            continue;
        }
        const uint64_t tau = a.out_scores ? 0ull : S.st.tau;
        emit_round(score, valid, row, a.n, qi, a.out_scores, topk_keys, &S.st, tau, a.smallest);
        if (!a.out_scores && a.mid_compact) {
            __syncthreads();
            topk_maybe_compact(topk_keys, &S.st, a.k, a.cap);
        }
    }
    if (LISTS)
        finish_wave_lists(a, list, thr, topk_keys, S, qi);
    else if (!a.out_scores)
        finish_topk(a, topk_keys, S, qi);
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

// Each thread scores one row per round (q4_row_dotf); the query digit
// planes are permuted to the nibble order (q4_perm_pos).
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
        if (valid) dotf = q4_row_dotf(packed + row * a.pitch, scales + row * a.nb, a.nb, qh, ql);
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
                               int8_t* hi, int8_t* lo, QConst* qc, uint64_t* tau, int* bcnt, hipStream_t s) {
    hipLaunchKernelGGL(query_encode_kernel, dim3(nq), dim3(256), 0, s, q, d, pitch, e16, c8, hi, lo, qc, tau, bcnt);
    return hipGetLastError();
}

hipError_t launch_query_encode_shadow(const uint16_t* q, int nq, int d, int spitch, int op, const ShadowInfo* info,
                                      int8_t* c8, int8_t* hi, int8_t* lo, QConst* qc, float* qb, uint64_t* tau,
                                      int* bcnt, hipStream_t s) {
    if (d % 32 != 0 || d > kMaxQueryDim || spitch < d) return hipErrorInvalidValue;
    hipLaunchKernelGGL(query_encode_shadow_kernel, dim3(nq), dim3(256), 0, s, q, d, spitch, op, info, c8, hi, lo, qc,
                       qb, tau, bcnt);
    return hipGetLastError();
}

bool q8_scan_coalesced(int pitch) {
    const int chunks = pitch / 16;
    return pitch % 16 == 0 && (chunks == 4 || chunks == 8 || chunks == 12 || chunks == 16 || chunks == 24 ||
                               chunks == 32 || chunks == 48 || chunks == 64);
}

template <int OP>
static hipError_t launch_q8_op(const ScanArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    const int chunks = a.pitch / 16;
    // the list path's merges use 64 LDS keys per wave
    if (a.wave_lists && !a.out_scores && lds < 256 * sizeof(uint64_t)) return hipErrorInvalidValue;
#define MANTA_Q8(LL, CC)                                                                           \
    if (chunks == (LL) * (CC)) {                                                                   \
        if (a.wave_lists && !a.out_scores)                                                         \
            hipLaunchKernelGGL((q8_scan_kernel<OP, LL, CC, true>), grid, dim3(256), lds, s, a);  \
        else                                                                                       \
            hipLaunchKernelGGL((q8_scan_kernel<OP, LL, CC, false>), grid, dim3(256), lds, s, a); \
        return hipGetLastError();                                                                  \
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
        case OP_DOT16: return launch_q8_op<OP_DOT16>(a, grid, lds, s);
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
