// q4_common.hpp -- the exact q4 score of one (query, row) pair under the
// packed contract, shared by the streaming q4 scan (lane = row), the
// rescoring of int8-shadow survivors (select kernel) and the shadow scan's
// region compaction.
//
// Contract (reference semantics it stands in for: dotRows / cosineRows /
// l2DistanceRows, runtime/backend/tensor_ops.go:1366-1490): per 32-element
// block b the exact integer sum acc_b of nibble codes times E16 query codes,
// dot = fma chain over the blocks of f16scale_b * f32(acc_b), qd = dot * qs,
// then the op's epilogue.
#pragma once

#include "device_common.hpp"
#include "kernels.hpp"

namespace manta {

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

// fma chain over the nb blocks of one packed row (16 bytes of nibbles and
// one f16 scale per block) against E16 digit planes qh / ql in the q4 order
// ([c0 c2 c4 c6 c1 c3 c5 c7] per 8 columns).  Nibbles become 16x-scaled
// int8 lanes: (w << 4) & 0xF0F0F0F0 holds the even nibbles of w as 16*code,
// w & 0xF0F0F0F0 the odd ones, so both digit sums are 16x the true ones and
// acc = 16*sh + sl/16 is exact.
__device__ __forceinline__ int q4_block_acc(v4i w, const int* qh, const int* ql) {
    int sh = 0, sl = 0;
    const int ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int even = (ws[j] << 4) & (int)0xF0F0F0F0;
        const int odd = ws[j] & (int)0xF0F0F0F0;
        sh = __builtin_amdgcn_sdot4(even, qh[2 * j], sh, false);
        sh = __builtin_amdgcn_sdot4(odd, qh[2 * j + 1], sh, false);
        sl = __builtin_amdgcn_sdot4(even, ql[2 * j], sl, false);
        sl = __builtin_amdgcn_sdot4(odd, ql[2 * j + 1], sl, false);
    }
    return (sh * 16) + (sl >> 4);
}

__device__ __forceinline__ float q4_row_dotf(const uint8_t* prow, const uint16_t* srow, int nb, const int* qh,
                                             const int* ql) {
    const v4i* rp = (const v4i*)prow;
    float dotf = 0.0f;
    for (int b = 0; b < nb; b++) dotf = __fmaf_rn(h2f(srow[b]), (float)q4_block_acc(rp[b], qh + 8 * b, ql + 8 * b), dotf);
    return dotf;
}

__device__ inline float q4_finish_op(int op, float dotf, const QConst& k, float dn, float d2) {
    if (op == OP_DOT) return q4_finish<OP_DOT>(dotf, k, 0.0f, 0.0f);
    if (op == OP_COSINE) return q4_finish<OP_COSINE>(dotf, k, dn, 0.0f);
    return q4_finish<OP_L2>(dotf, k, 0.0f, d2);
}

// Exact score of row `row` of a q4 matrix ([n][d/2] bytes, f16 [n][d/32]
// scales) for one E16-encoded query; op is OP_DOT, OP_COSINE or OP_L2.
__device__ inline float q4_exact_score(int op, const uint8_t* codes, const uint16_t* scales, const float* dnorm,
                                       const float* dd, int d, int64_t row, const int* qh, const int* ql,
                                       const QConst& k) {
    const int nb = d / 32;
    const float dotf = q4_row_dotf(codes + row * (d / 2), scales + row * nb, nb, qh, ql);
    return q4_finish_op(op, dotf, k, op == OP_COSINE ? dnorm[row] : 0.0f, op == OP_L2 ? dd[row] : 0.0f);
}

// Threshold on the int8 shadow's pre-score p = scale_r * acc from a key of
// exact scores: a row whose exact score reaches key_score(tk) has
// p >= (ts - m) * f (largest first; (ts + m) * f and <= for smallest first),
// with m the query's error margin and f its score -> pre-score factor.  The
// margin carries an absolute slack far above the f32 roundings of this
// formula, and loosen_* covers the relative ones.  No threshold lets
// everything through.
__device__ __forceinline__ float shadow_bound(uint64_t tk, float m, float f, bool smallest) {
    if (!tk) return smallest ? __builtin_inff() : -__builtin_inff();
    const float ts = key_score(tk, smallest);
    if (smallest) {
        const float x = fmul_rn(fadd_rn(ts, m), f);
        return x + __builtin_fabsf(x) * 9.5367431640625e-7f + 1e-30f;
    }
    const float x = fmul_rn(fsub_rn(ts, m), f);
    return x - __builtin_fabsf(x) * 9.5367431640625e-7f - 1e-30f;
}

}  // namespace manta
