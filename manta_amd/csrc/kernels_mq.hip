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

template <int OP, int ENC, int QG, int KS, int TJ>
__global__ __launch_bounds__(256) void mq_q8_kernel(MqArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int APITCH = KS * 32 + 16;  // bytes per A row in LDS (padded)
    constexpr int QPL = ENC == MQ_E8 ? 16 : (QG == 16 ? 8 : 4);  // queries per lane
    int8_t* arows = (int8_t*)smem;                          // [32][APITCH]
    TopKShared* st = (TopKShared*)(smem + 32 * APITCH);      // [QG]
    uint64_t* keys = (uint64_t*)(smem + 32 * APITCH + QG * sizeof(TopKShared));  // [QG][cap]
    __shared__ QConst qcs[32];
    __shared__ uint64_t tau_s[QG];  // max(local reservoir tau, global tau) per query
    __shared__ uint32_t cmask;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int half = lane >> 5;
    const int q0 = blockIdx.y * QG;
    const bool topk = a.out_scores == nullptr;

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
        }
    }
    __syncthreads();

    // ---- per-lane query slots
    // E8:  slot r (0..15) -> A row 8*(r/4) + 4*half + r%4 = query.
    // E16: slot u -> hi acc index r_hi, lo index r_hi + 4, query index.
    int slot_q[QPL];
    int slot_r[QPL];
#pragma unroll
    for (int u = 0; u < QPL; u++) {
        if (ENC == MQ_E8) {
            slot_r[u] = u;
            slot_q[u] = 8 * (u / 4) + 4 * half + (u % 4);
        } else {
            const int r = (u < 4) ? u : 8 + (u - 4);  // hi accumulators 0-3, 8-11
            slot_r[u] = r;
            const int i = 8 * (r / 4) + 4 * half + (r % 4);  // hi A row
            slot_q[u] = (i >> 4) * 8 + (i & 7);
        }
    }

    const int64_t range0 = (int64_t)blockIdx.x * a.rows_per_wg;
    int64_t range1 = range0 + a.rows_per_wg;
    if (range1 > a.n) range1 = a.n;
    constexpr int TILE = 4 * TJ * 32;

    for (int64_t t0 = range0; t0 < range1; t0 += TILE) {
        // thresholds for this tile (local reservoir or any workgroup's)
        float bound[QPL];
        uint64_t tau[QPL];
#pragma unroll
        for (int u = 0; u < QPL; u++) {
            const int qq = slot_q[u];
            const uint64_t tk = (topk && qq < QG) ? tau_s[qq] : 0ull;
            tau[u] = tk;
            if (!tk) {
                bound[u] = a.smallest ? __builtin_inff() : -__builtin_inff();
            } else {
                const float ts = key_score(tk, a.smallest);
                if (OP == OP_DOT) {
                    const float tt = fmul_rn(ts, 127.0f);
                    bound[u] = a.smallest ? loosen_up(tt) : loosen_down(tt);
                } else if (OP == OP_L2) {
                    const float t2 = fmul_rn(ts, ts);
                    bound[u] = a.smallest ? loosen_up(t2) : loosen_down(t2);
                } else {
                    bound[u] = a.smallest ? __builtin_inff() : -__builtin_inff();
                }
            }
        }

#pragma unroll
        for (int tj = 0; tj < TJ; tj++) {
            const int64_t rowblk = t0 + (int64_t)(wave * TJ + tj) * 32;
            const int64_t row = rowblk + (lane & 31);
            const bool rvalid = row < range1;
            // B fragments: 16 bytes of the candidate row per K step
            v4i b[KS];
            const int8_t* rp = a.codes + row * a.pitch + half * 16;
#pragma unroll
            for (int s = 0; s < KS; s++)
                b[s] = rvalid ? __builtin_nontemporal_load((const v4i*)(rp + s * 32)) : v4i{0, 0, 0, 0};
            v16i acc;
#pragma unroll
            for (int r = 0; r < 16; r++) acc[r] = 0;
#pragma unroll
            for (int s = 0; s < KS; s++) {
                const v4i av = *(const v4i*)(arows + (lane & 31) * APITCH + s * 32 + half * 16);
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b[s], acc, 0, 0, 0);
            }
            if (!rvalid) continue;
            const float scale = a.scales[row];
            float rowc = 0.0f;
            if (OP == OP_COSINE) rowc = a.dnorm[row];
            if (OP == OP_L2) rowc = a.dd[row];
#pragma unroll
            for (int u = 0; u < QPL; u++) {
                const int qq = slot_q[u];
                const int q = q0 + qq;
                if ((ENC == MQ_E16 && qq >= QG) || q >= a.nq) continue;
                const QConst kq = qcs[qq];
                float score;
                bool pass;
                if (OP == OP_DOT) {
                    float t = fmul_rn(fmul_rn(scale, (float)acc[slot_r[u]]), kq.a);
                    pass = a.smallest ? (t <= bound[u]) : (t >= bound[u]);
                    if (!topk) pass = true;
                    if (!pass) continue;
                    score = fdiv_rn(t, 127.0f);
                } else {
                    const float dotf = __fmaf_rn(256.0f, (float)acc[slot_r[u]], (float)acc[slot_r[u] + 4]);
                    const float qd = fmul_rn(fmul_rn(scale, kq.a), dotf);
                    if (OP == OP_COSINE) {
                        const float den = fmul_rn(kq.b, rowc);
                        score = den == 0.0f ? 0.0f : fdiv_rn(qd, den);
                    } else {
                        const float t = fadd_rn(kq.c, rowc);
                        float dist2 = fsub_rn(t, fmul_rn(2.0f, qd));
                        pass = a.smallest ? (dist2 <= bound[u]) : (dist2 >= bound[u]);
                        if (!topk) pass = true;
                        if (!pass) continue;
                        dist2 = dist2 < 0.0f ? 0.0f : dist2;
                        score = fsqrt_rn(dist2);
                    }
                }
                if (!topk) {
                    a.out_scores[(int64_t)q * a.n + row] = score;
                    continue;
                }
                const uint64_t key = make_key(score, (uint32_t)row, a.smallest);
                if (key > tau[u]) {
                    const int pos = atomicAdd(&st[qq].cnt, 1);
                    keys[(int64_t)qq * a.cap + pos] = key;
                }
            }
        }
        if (!topk) continue;
        // ---- keep every reservoir able to take the next tile
        __syncthreads();
        if (tid == 0) {
            uint32_t m = 0;
            for (int qq = 0; qq < QG; qq++)
                if (st[qq].cnt + TILE > a.cap) m |= 1u << qq;
            cmask = m;
        }
        __syncthreads();
        const uint32_t m = cmask;
        for (int qq = 0; qq < QG; qq++) {
            if (!(m & (1u << qq))) continue;
            topk_compact(keys + (int64_t)qq * a.cap, &st[qq], a.k);
            if (tid == 0 && st[qq].tau && q0 + qq < a.nq) atomicMax(&a.gtau[q0 + qq], st[qq].tau);
        }
        if (tid < QG && q0 + tid < a.nq) {
            const uint64_t g = __hip_atomic_load(&a.gtau[q0 + tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            tau_s[tid] = st[tid].tau > g ? st[tid].tau : g;
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

template <int OP, int ENC, int QG>
static hipError_t launch_mq_ks(const MqArgs& a, dim3 grid, size_t lds, hipStream_t s, int ks) {
#define MANTA_MQ(KSV, TJV)                                                                     \
    if (ks == (KSV)) {                                                                         \
        hipLaunchKernelGGL((mq_q8_kernel<OP, ENC, QG, KSV, TJV>), grid, dim3(256), lds, s, a); \
        return hipGetLastError();                                                              \
    }
    MANTA_MQ(2, 4)
    MANTA_MQ(4, 4)
    MANTA_MQ(8, 2)
    MANTA_MQ(12, 1)
    MANTA_MQ(16, 1)
#undef MANTA_MQ
    return hipErrorInvalidValue;
}

int mq_tile_rows(int ks) {
    const int tj = ks <= 4 ? 4 : (ks <= 8 ? 2 : 1);
    return 4 * tj * 32;
}

bool mq_supported_ks(int ks) { return ks == 2 || ks == 4 || ks == 8 || ks == 12 || ks == 16; }

hipError_t launch_mq_q8(int op, int qg, const MqArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    const int ks = a.pitch / 32;
    if (op == OP_DOT) return launch_mq_ks<OP_DOT, MQ_E8, 32>(a, grid, lds, s, ks);
    if (op == OP_COSINE) {
        if (qg == 16) return launch_mq_ks<OP_COSINE, MQ_E16, 16>(a, grid, lds, s, ks);
        return launch_mq_ks<OP_COSINE, MQ_E16, 8>(a, grid, lds, s, ks);
    }
    if (qg == 16) return launch_mq_ks<OP_L2, MQ_E16, 16>(a, grid, lds, s, ks);
    return launch_mq_ks<OP_L2, MQ_E16, 8>(a, grid, lds, s, ks);
}

hipError_t launch_mq_clear(unsigned long long* gtau, int nq, hipStream_t s) {
    hipLaunchKernelGGL(mq_clear_kernel, dim3((nq + 255) / 256), dim3(256), 0, s, gtau, nq);
    return hipGetLastError();
}

}  // namespace manta
