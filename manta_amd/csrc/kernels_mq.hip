// kernels_mq.hip -- many queries against one shared q8 candidate matrix
// ([Q,D] x [N,D]) on the i8 matrix cores of gfx950.
//
// Workgroup = 4 waves; grid = (row ranges, query groups).  The group's query
// codes sit in LDS as the A operand of v_mfma_i32_32x32x32_i8 (32 "rows" =
// queries or query digits); each wave streams TJ blocks of 32 candidate rows
// per tile straight from HBM as the B operand (16 bytes per lane per
// 32-wide K step), so every candidate byte is loaded once per query group.
// With the candidate on the output column, a lane ends a tile holding one
// candidate row against 16 A rows:
//   E8 (dot, 32 queries per group)      : 16 queries per lane;
//   E16 (cosine / l2, 8 or 16 queries)  : A rows [hi q0-7 | lo q0-7 | hi
//        q8-15 | lo q8-15], so a query's hi and lo sums land in the same lane
//        (acc[r] and acc[r+4]) and combine exactly as fma(256, hi, lo).
// The epilogue evaluates a cheap monotone pre-score (t = (s*acc)*qmax for
// dot, dist^2 for l2) against a conservative per-query bound derived from
// the current threshold key, and only survivors get the exact score and key
// (the same f32 formulas as the streaming kernels and the CPU oracle).
// Keys go to per-query LDS reservoirs (radix-select compaction); each
// compaction raises a per-query global threshold (agent-scope atomic max)
// that every workgroup filters with.  Each workgroup finally writes k keys
// per query; topk_merge_kernel reduces them.  Row ranges are a multiple of 8
// long in blocks, so the workgroups of different query groups that share a
// range share an XCD (and its L2).
#include "device_common.hpp"
#include "kernels.hpp"

namespace manta {

typedef int v16i __attribute__((ext_vector_type(16)));

enum { MQ_E8 = 0, MQ_E16 = 1 };

// Conservative pre-score bounds from a threshold key.  Survivors of the
// bound are re-checked with the exact key, so the bound only has to be
// loose on the safe side (relative 2^-20 covers every rounding in t and
// dist^2).
__device__ __forceinline__ float loosen_down(float x) {
    return x - __builtin_fabsf(x) * 9.5367431640625e-7f - 1e-30f;
}
__device__ __forceinline__ float loosen_up(float x) {
    return x + __builtin_fabsf(x) * 9.5367431640625e-7f + 1e-30f;
}

// Pre-score bound of one query from its threshold key: dot compares s*acc
// against (tau*127)/qmax, l2 compares dist^2 against tau^2; no threshold (or
// cosine) lets everything through.
template <int OP>
__device__ __forceinline__ float mq_bound(uint64_t tk, const QConst& qc, int smallest) {
    const float open = smallest ? __builtin_inff() : -__builtin_inff();
    if (!tk) return open;
    const float ts = key_score(tk, smallest);
    if (OP == OP_DOT) {
        const float tt = fdiv_rn(fmul_rn(ts, 127.0f), qc.a);
        return smallest ? loosen_up(tt) : loosen_down(tt);
    }
    if (OP == OP_L2) {
        const float t2 = fmul_rn(ts, ts);
        return smallest ? loosen_up(t2) : loosen_down(t2);
    }
    return open;
}

template <int OP, int ENC, int QG, int KS, int TJ, bool SMALL, bool TOPK>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void mq_q8_kernel(MqArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int APITCH = KS * 32 + 16;  // bytes per A row in LDS (padded)
    constexpr int QPL = ENC == MQ_E8 ? 16 : (QG == 16 ? 8 : 4);  // queries per lane
    int8_t* arows = (int8_t*)smem;                          // [32][APITCH]
    TopKShared* st = (TopKShared*)(smem + 32 * APITCH);      // [QG]
    uint64_t* keys = (uint64_t*)(smem + 32 * APITCH + QG * sizeof(TopKShared));  // [QG][cap]
    __shared__ QConst qcs[32];
    __shared__ uint64_t tau_s[QG];  // max(local reservoir tau, global tau) per query
    __shared__ float bound_s[QG];   // pre-score bound derived from tau_s
    __shared__ uint32_t cmask;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int half = lane >> 5;
    const int q0 = blockIdx.y * QG;
    constexpr bool topk = TOPK;

    // ---- A rows: query codes (E8) or digit planes (E16)
    for (int idx = tid; idx < 32 * (KS * 2); idx += 256) {
        const int i = idx / (KS * 2);
        const int seg = idx % (KS * 2);  // 16-byte segment of the row
        int q = -1;
        const int8_t* src = nullptr;
        if (ENC == MQ_E8) {
            q = q0 + i;
            src = a.qc8;
        } else {
            const int blk = i >> 3;  // 0: hi 0-7, 1: lo 0-7, 2: hi 8-15, 3: lo 8-15
            const int qq = (blk >> 1) * 8 + (i & 7);
            if (qq < QG) {
                q = q0 + qq;
                src = (blk & 1) ? a.qlo : a.qhi;
            }
        }
        v4i v = v4i{0, 0, 0, 0};
        if (src && q < a.nq && seg * 16 < a.pitch) v = *(const v4i*)(src + (int64_t)q * a.pitch + seg * 16);
        *(v4i*)(arows + i * APITCH + seg * 16) = v;
    }
    if (tid < 32) qcs[tid] = (q0 + tid < a.nq && tid < QG) ? a.qconst[q0 + tid] : QConst{0, 0, 0, 0};
    if (topk) {
        for (int q = tid; q < QG; q += 256) {
            st[q].cnt = 0;
            st[q].tau = 0;
            tau_s[q] = 0;
            bound_s[q] = SMALL ? __builtin_inff() : -__builtin_inff();
        }
    }
    __syncthreads();

    // ---- per-lane query slots
    // E8:  slot u (0..15) = accumulator u = A row 8*(u/4) + 4*half + u%4 = query.
    // E16: slot u -> hi accumulator r = (u < 4 ? u : u + 4), lo accumulator
    //      r + 4, hi A row i = 8*(r/4) + 4*half + r%4, query (i/16)*8 + i%8.
    auto slot_r = [](int u) { return ENC == MQ_E8 ? u : (u < 4 ? u : u + 4); };
    auto slot_q = [&](int u) {
        const int r = slot_r(u);
        const int i = 8 * (r / 4) + 4 * half + (r % 4);
        return ENC == MQ_E8 ? i : (i >> 4) * 8 + (i & 7);
    };
    uint32_t live_mask = 0;
#pragma unroll
    for (int u = 0; u < QPL; u++) {
        const int qq = slot_q(u);
        if (qq < QG && q0 + qq < a.nq) live_mask |= 1u << u;
    }

    const int64_t range0 = (int64_t)blockIdx.x * a.rows_per_wg;
    int64_t range1 = range0 + a.rows_per_wg;
    if (range1 > a.n) range1 = a.n;
    constexpr int TILE = 4 * TJ * 32;

    // B fragments (16 bytes of a candidate row per K step) of the next tile
    // are loaded while the current one is multiplied.
    v4i bn[TJ][KS];
    float sn[TJ], cn[TJ];  // scale and |d| or |d|^2 of the prefetched rows
    auto load_tile = [&](int64_t t0) {
#pragma unroll
        for (int tj = 0; tj < TJ; tj++) {
            const int64_t row = t0 + (int64_t)(wave * TJ + tj) * 32 + (lane & 31);
            const bool ok = row < range1;
            const int64_t rr = ok ? row : 0;
            const int8_t* rp = a.codes + rr * a.pitch + half * 16;
#pragma unroll
            for (int s = 0; s < KS; s++)
                bn[tj][s] = ok ? *(const v4i*)(rp + s * 32) : v4i{0, 0, 0, 0};
            sn[tj] = a.scales[rr];
            cn[tj] = OP == OP_COSINE ? a.dnorm[rr] : (OP == OP_L2 ? a.dd[rr] : 0.0f);
        }
    };
    if (range0 < range1) load_tile(range0);
    // shared thresholds are read one tile ahead of their use
    uint64_t gnext = 0;
    if (topk && tid < QG && q0 + tid < a.nq)
        gnext = __hip_atomic_load(&a.gtau[q0 + tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    for (int64_t t0 = range0; t0 < range1; t0 += TILE) {
        float sc[TJ], cc[TJ];
#pragma unroll
        for (int tj = 0; tj < TJ; tj++) {
            sc[tj] = sn[tj];
            cc[tj] = cn[tj];
        }

        // per-slot filter bounds (computed once per query per tile, in LDS)
        float bound[QPL];
#pragma unroll
        for (int u = 0; u < QPL; u++) bound[u] = bound_s[slot_q(u) < QG ? slot_q(u) : 0];

        // MFMA phase: independent accumulator chains (TJ row blocks, and the
        // K steps split in two for long rows) so the matrix pipe never waits
        // on its own previous result.
        constexpr int NC = (KS >= 8) ? 2 : 1;
        v16i acc[TJ][NC];
#pragma unroll
        for (int tj = 0; tj < TJ; tj++)
#pragma unroll
            for (int c = 0; c < NC; c++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[tj][c][r] = 0;
#pragma unroll
        for (int s = 0; s < KS; s++) {
            const v4i av = *(const v4i*)(arows + (lane & 31) * APITCH + s * 32 + half * 16);
#pragma unroll
            for (int tj = 0; tj < TJ; tj++)
                acc[tj][s % NC] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bn[tj][s], acc[tj][s % NC], 0, 0, 0);
        }
        // the fragments are consumed: start the next tile's loads now so they
        // overlap this tile's epilogue and reservoir upkeep
        if (t0 + TILE < range1) load_tile(t0 + TILE);

#pragma unroll
        for (int tj = 0; tj < TJ; tj++) {
            const int64_t row = t0 + (int64_t)(wave * TJ + tj) * 32 + (lane & 31);
            if (row >= range1) continue;
            v16i accs = acc[tj][0];
            if (NC > 1) accs += acc[tj][NC - 1];
            const float scale = sc[tj];
            const float rowc = cc[tj];
            // pre-scores: dot s*acc, l2 dist^2, cosine q.d (exact f32 steps)
            auto pre_of = [&](int hi, int lo, int qq) {
                if (OP == OP_DOT) return fmul_rn(scale, (float)hi);
                const float dotf = __fmaf_rn(256.0f, (float)hi, (float)lo);
                const float qd = fmul_rn(fmul_rn(scale, qcs[qq].a), dotf);
                return OP == OP_L2 ? fsub_rn(fadd_rn(qcs[qq].c, rowc), fmul_rn(2.0f, qd)) : qd;
            };
            uint32_t pmask = 0;
#pragma unroll
            for (int u = 0; u < QPL; u++) {
                const int r = slot_r(u);
                const float p = pre_of(accs[r], ENC == MQ_E8 ? 0 : accs[r + 4], slot_q(u) < QG ? slot_q(u) : 0);
                const bool keep = !topk || (SMALL ? !(p > bound[u]) : !(p < bound[u]));
                if (keep) pmask |= 1u << u;
            }
            pmask &= live_mask;
            // exact scores for the survivors only (rare once thresholds settle)
            while (pmask) {
                const int u = __builtin_ctz(pmask);
                pmask &= pmask - 1;
                int hi = accs[slot_r(0)], lo = ENC == MQ_E8 ? 0 : accs[slot_r(0) + 4];
#pragma unroll
                for (int w = 1; w < QPL; w++) {
                    hi = (u == w) ? accs[slot_r(w)] : hi;
                    if (ENC != MQ_E8) lo = (u == w) ? accs[slot_r(w) + 4] : lo;
                }
                const int r0 = slot_r(u);
                const int i0 = 8 * (r0 / 4) + 4 * half + (r0 % 4);
                const int qq = ENC == MQ_E8 ? i0 : (i0 >> 4) * 8 + (i0 & 7);
                const float v = pre_of(hi, lo, qq);
                float score;
                if (OP == OP_DOT) {
                    score = fdiv_rn(fmul_rn(v, qcs[qq].a), 127.0f);
                } else if (OP == OP_COSINE) {
                    const float den = fmul_rn(qcs[qq].b, rowc);
                    score = den == 0.0f ? 0.0f : fdiv_rn(v, den);
                } else {
                    score = fsqrt_rn(v < 0.0f ? 0.0f : v);
                }
                if (!topk) {
                    a.out_scores[(int64_t)(q0 + qq) * a.n + row] = score;
                    continue;
                }
                const uint64_t key = make_key(score, (uint32_t)row, SMALL);
                if (key > tau_s[qq]) {
                    const int pos = atomicAdd(&st[qq].cnt, 1);
                    keys[(int64_t)qq * a.cap + pos] = key;
                }
            }
        }
        if (!topk) continue;
        // ---- keep every reservoir able to take the next tile
        __syncthreads();
        if (tid < 64) {
            const bool need = tid < QG && st[tid].cnt + TILE > a.cap;
            const uint64_t m = __ballot(need);
            if (tid == 0) cmask = (uint32_t)m;
        }
        __syncthreads();
        const uint32_t m = cmask;
        for (int qq = 0; qq < QG; qq++) {
            if (!(m & (1u << qq))) continue;
            topk_compact(keys + (int64_t)qq * a.cap, &st[qq], a.k);
            if (tid == 0 && st[qq].tau && q0 + qq < a.nq) atomicMax(&a.gtau[q0 + qq], st[qq].tau);
        }
        if (tid < QG && q0 + tid < a.nq) {
            const uint64_t tk = st[tid].tau > gnext ? st[tid].tau : gnext;
            tau_s[tid] = tk;
            bound_s[tid] = mq_bound<OP>(tk, qcs[tid], SMALL);
            gnext = __hip_atomic_load(&a.gtau[q0 + tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
    }
    if (!topk) return;
    // ---- publish k keys per query
    for (int qq = 0; qq < QG; qq++) {
        if (q0 + qq >= a.nq) break;
        topk_compact(keys + (int64_t)qq * a.cap, &st[qq], a.k);
        uint64_t* dst = a.partial + ((int64_t)(q0 + qq) * gridDim.x + blockIdx.x) * a.k;
        const int c = st[qq].cnt;
        for (int i = tid; i < a.k; i += 256) dst[i] = i < c ? keys[(int64_t)qq * a.cap + i] : 0ull;
        if (tid == 0 && st[qq].tau) atomicMax(&a.gtau[q0 + qq], st[qq].tau);
        __syncthreads();
    }
}

// Zero the per-query global thresholds before a call (a fill kernel, not a
// memset node, so a captured graph replays it reliably).
__global__ void mq_clear_kernel(unsigned long long* gtau, int nq) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < nq) gtau[i] = 0ull;
}

// ----------------------------------------------------------------- hosts

template <int OP, int ENC, int QG, bool SMALL, bool TOPK>
static hipError_t launch_mq_ks(const MqArgs& a, dim3 grid, size_t lds, hipStream_t s, int ks) {
#define MANTA_MQ(KSV, TJV)                                                                                   \
    if (ks == (KSV)) {                                                                                       \
        hipLaunchKernelGGL((mq_q8_kernel<OP, ENC, QG, KSV, TJV, SMALL, TOPK>), grid, dim3(256), lds, s, a); \
        return hipGetLastError();                                                                            \
    }
    MANTA_MQ(2, 4)
    MANTA_MQ(4, 4)
    MANTA_MQ(8, 2)
    MANTA_MQ(12, 1)
    MANTA_MQ(16, 1)
#undef MANTA_MQ
    return hipErrorInvalidValue;
}

template <int OP, int ENC, int QG>
static hipError_t launch_mq_mode(const MqArgs& a, dim3 grid, size_t lds, hipStream_t s, int ks) {
    if (a.out_scores) return launch_mq_ks<OP, ENC, QG, false, false>(a, grid, lds, s, ks);
    if (a.smallest) return launch_mq_ks<OP, ENC, QG, true, true>(a, grid, lds, s, ks);
    return launch_mq_ks<OP, ENC, QG, false, true>(a, grid, lds, s, ks);
}

int mq_tile_rows(int ks) {
    const int tj = ks <= 4 ? 4 : (ks <= 8 ? 2 : 1);
    return 4 * tj * 32;
}

bool mq_supported_ks(int ks) { return ks == 2 || ks == 4 || ks == 8 || ks == 12 || ks == 16; }

hipError_t launch_mq_q8(int op, int qg, const MqArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    const int ks = a.pitch / 32;
    if (op == OP_DOT) return launch_mq_mode<OP_DOT, MQ_E8, 32>(a, grid, lds, s, ks);
    if (op == OP_COSINE) {
        if (qg == 16) return launch_mq_mode<OP_COSINE, MQ_E16, 16>(a, grid, lds, s, ks);
        return launch_mq_mode<OP_COSINE, MQ_E16, 8>(a, grid, lds, s, ks);
    }
    if (qg == 16) return launch_mq_mode<OP_L2, MQ_E16, 16>(a, grid, lds, s, ks);
    return launch_mq_mode<OP_L2, MQ_E16, 8>(a, grid, lds, s, ks);
}

hipError_t launch_mq_clear(unsigned long long* gtau, int nq, hipStream_t s) {
    hipLaunchKernelGGL(mq_clear_kernel, dim3((nq + 255) / 256), dim3(256), 0, s, gtau, nq);
    return hipGetLastError();
}

}  // namespace manta
