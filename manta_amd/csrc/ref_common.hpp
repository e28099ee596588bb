// ref_common.hpp -- the reference's score arithmetic on the device, and the
// error bounds that tie the quantized-query scan scores to it.
//
// Reference semantics (runtime/backend/tensor_ops.go):
//   dotRows        :1366-1396  f32 sum over columns in order, each product
//                              and each sum rounded on its own;
//   cosineRows     :1398-1456  f64 dot and norms accumulated in column order,
//                              denom = sqrt(qn) * sqrt(dn), 0 when denom is 0,
//                              dot / denom narrowed to f32;
//   l2DistanceRows :1458-1490  f32 difference, f64 square-sum in column
//                              order, sqrt, narrowed to f32.
// The values are those an f32-backed reference q8 / q4 tensor holds for a
// packed element: fl32(code * scale) (the grid stores q*scale in f32,
// runtime/embedding_trainer.go:3753-3762); q4: code * f16 scale (exact).
// Queries are f16 widened to f32 (exact).
//
// Every f64 product in these loops is exact (two values of at most 24
// significant bits), so an f64 fma equals the reference's multiply-then-add.
#pragma once

#include "device_common.hpp"

namespace manta {

typedef unsigned __int128 u128;

// x > 0, finite: x = m * 2^e with m < 2^53.
__device__ __forceinline__ void dsplit(double x, uint64_t& m, int& e) {
    const uint64_t b = (uint64_t)__double_as_longlong(x);
    const int ex = (int)((b >> 52) & 0x7FF);
    m = b & ((1ull << 52) - 1);
    if (ex == 0) {
        e = -1074;
    } else {
        m |= 1ull << 52;
        e = ex - 1075;
    }
}

// Sign of X*2^ex - (M*2^em)^2, exactly (X < 2^53, M < 2^55).
__device__ inline int cmp_square(uint64_t X, int ex, uint64_t M, int em) {
    const u128 P = (u128)M * M;  // < 2^110
    const int sh = ex - 2 * em;  // compare X * 2^sh with P
    if (sh >= 0) {
        const int lx = 64 - __builtin_clzll(X);
        if (lx + sh > 120) return 1;  // X * 2^sh >= 2^120 > P
        const u128 L = (u128)X << sh;
        return L > P ? 1 : (L < P ? -1 : 0);
    }
    const int lp = 128 - (int)(P >> 64 ? __builtin_clzll((uint64_t)(P >> 64)) : 64 + __builtin_clzll((uint64_t)P));
    if (lp - sh > 120) return -1;  // P * 2^-sh >= 2^120 > X
    const u128 R = P << (-sh);
    const u128 L = (u128)X;
    return L > R ? 1 : (L < R ? -1 : 0);
}

__device__ __forceinline__ double dnext_up(double y) {
    return __longlong_as_double(__double_as_longlong(y) + 1);  // y > 0
}
__device__ __forceinline__ double dnext_down(double y) {
    return __longlong_as_double(__double_as_longlong(y) - 1);  // y > 0
}

// Correctly rounded f64 square root (Go's math.Sqrt): the hardware result,
// checked against the two rounding midpoints around it with exact integer
// arithmetic and moved by an ulp until it lies between them (a square root
// of a double is never a midpoint, so there is no tie).
__device__ inline double sqrt_rn(double x) {
    double y = __builtin_sqrt(x);
    if (!(x > 0.0) || !(x < __builtin_inf())) return y;
    uint64_t X;
    int ex;
    dsplit(x, X, ex);
    for (int it = 0; it < 4; it++) {
        uint64_t Y;
        int ey;
        dsplit(y, Y, ey);  // y >= 2^-537: normal, Y >= 2^52
        if (cmp_square(X, ex, 2 * Y + 1, ey - 1) > 0) {
            y = dnext_up(y);
            continue;
        }
        const bool low = Y == (1ull << 52) ? cmp_square(X, ex, 4 * Y - 1, ey - 2) < 0
                                           : cmp_square(X, ex, 2 * Y - 1, ey - 1) < 0;
        if (low) {
            y = dnext_down(y);
            continue;
        }
        break;
    }
    return y;
}

// Correctly rounded f64 division: of the hardware quotient and its two
// neighbours, the one with the smallest exact remainder a - c*b (an fma
// computes it exactly for candidates within an ulp of a/b; there are no
// ties in division).
__device__ inline double div_rn(double a, double b) {
    const double q = a / b;
    if (!(q != 0.0) || !__builtin_isfinite(q) || !__builtin_isfinite(a) || !__builtin_isfinite(b)) return q;
    // the neighbours of a nonzero finite q: one step of its bit pattern
    const long long qb = __double_as_longlong(q);
    const double qu = __longlong_as_double(q > 0.0 ? qb + 1 : qb - 1);
    const double qd = __longlong_as_double(q > 0.0 ? qb - 1 : qb + 1);
    const double r = __builtin_fabs(__builtin_fma(-q, b, a));
    const double ru = __builtin_fabs(__builtin_fma(-qu, b, a));
    const double rd = __builtin_fabs(__builtin_fma(-qd, b, a));
    if (ru < r) return qu;
    if (rd < r) return qd;
    return q;
}

// The reference's f64 norm term sqrt(sum x^2), summed in column order.
__device__ inline double ref_sqrt_norm(const float* x, int d) {
    double s = 0.0;
    for (int c = 0; c < d; c++) s = __fma_rn((double)x[c], (double)x[c], s);
    return sqrt_rn(s);
}

// Accumulator of one reference score, fed the (query, value) pairs of a row
// in column order.
template <int OP>
struct RefAcc {
    float f = 0.0f;   // dotRows
    double s = 0.0;   // cosineRows dot / l2DistanceRows square-sum
    __device__ __forceinline__ void add(float q, float v) {
        if (OP == OP_DOT) {
            f = fadd_rn(f, fmul_rn(q, v));
        } else if (OP == OP_COSINE) {
            s = __fma_rn((double)q, (double)v, s);
        } else {
            const float df = fsub_rn(q, v);
            s = __fma_rn((double)df, (double)df, s);
        }
    }
    // sqn / sqd: the query's and the row's f64 norm terms (cosine only)
    __device__ __forceinline__ float finish(double sqn, double sqd) const {
        if (OP == OP_DOT) return f;
        if (OP == OP_COSINE) {
            const double den = dmul_rn(sqn, sqd);
            return den == 0.0 ? 0.0f : (float)div_rn(s, den);
        }
        return (float)sqrt_rn(s);
    }
};

// Reference score of q8 row `row` (pitch bytes, 16-byte aligned, d codes,
// f32 scale s) against the f32 query qf[0..d): ref_acc_q8 runs the
// sequential sum, ref_score_q8 also finishes it.  The row's bytes arrive 128
// at a time (eight 16-byte loads), the next 128 loaded while the current
// ones are summed.
template <int OP>
__device__ __forceinline__ RefAcc<OP> ref_acc_q8(const float* qf, const int8_t* row, float s, int d) {
    RefAcc<OP> acc;
    // (loads past the row's last 16 bytes re-read them: no branch between
    // the loads, so they all go out at once; those values are never used)
    const int last = (d - 1) & ~15;
    v4i w[8], wn[8];
    auto load = [&](v4i (&dst)[8], int c0) {
#pragma unroll
        for (int j = 0; j < 8; j++) dst[j] = *(const v4i*)(row + (c0 + 16 * j < last ? c0 + 16 * j : last));
    };
    auto sum = [&](const v4i (&g)[8], int c0) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int ws[4] = {g[j].x, g[j].y, g[j].z, g[j].w};
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int c = c0 + 16 * j + e;
                if (c >= d) break;
                const int code = (ws[e >> 2] << (24 - 8 * (e & 3))) >> 24;
                acc.add(qf[c], fmul_rn((float)code, s));
            }
        }
    };
    // two buffers in turn, so a sum waits only for its own group's loads
    load(w, 0);
    for (int c0 = 0; c0 < d; c0 += 256) {
        if (c0 + 128 < d) load(wn, c0 + 128);
        sum(w, c0);
        if (c0 + 128 >= d) break;
        if (c0 + 256 < d) load(w, c0 + 256);
        sum(wn, c0 + 128);
    }
    return acc;
}
template <int OP>
__device__ inline float ref_score_q8(const float* qf, const int8_t* row, float s, int d, double sqn, double sqd) {
    return ref_acc_q8<OP>(qf, row, s, d).finish(sqn, sqd);
}

// Reference score of a q4 row (d/2 bytes of nibbles, low nibble first, and
// d/32 f16 block scales; d % 32 == 0): the sum (ref_acc_q4) and the finished
// score (ref_score_q4).  Blocks arrive four at a time, the next four loaded
// while the current ones are summed.
template <int OP>
__device__ __forceinline__ RefAcc<OP> ref_acc_q4(const float* qf, const uint8_t* prow, const uint16_t* srow, int d) {
    RefAcc<OP> acc;
    const int nb = d / 32;
    v4i w[4], wn[4];
    uint16_t sb[4], sbn[4];  // raw f16 scales: converted where used, so a
                             // prefetch is never waited for early
    // (blocks past the row's last re-read it: no branch between the loads)
    auto load = [&](v4i (&dw)[4], uint16_t (&ds)[4], int b0) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int b = b0 + j < nb ? b0 + j : nb - 1;
            dw[j] = ((const v4i*)prow)[b];
            ds[j] = srow[b];
        }
    };
    auto sum = [&](const v4i (&g)[4], const uint16_t (&gs)[4], int b0) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (b0 + j >= nb) break;
            const int ws[4] = {g[j].x, g[j].y, g[j].z, g[j].w};
            const float sj = h2f(gs[j]);
#pragma unroll
            for (int e = 0; e < 32; e++) {
                const int code = (ws[e >> 3] << (28 - 4 * (e & 7))) >> 28;
                acc.add(qf[(b0 + j) * 32 + e], fmul_rn((float)code, sj));
            }
        }
    };
    // two buffers in turn, so a sum waits only for its own blocks' loads
    load(w, sb, 0);
    for (int b0 = 0; b0 < nb; b0 += 8) {
        if (b0 + 4 < nb) load(wn, sbn, b0 + 4);
        sum(w, sb, b0);
        if (b0 + 4 >= nb) break;
        if (b0 + 8 < nb) load(w, sb, b0 + 8);
        sum(wn, sbn, b0 + 4);
    }
    return acc;
}
template <int OP>
__device__ inline float ref_score_q4(const float* qf, const uint8_t* prow, const uint16_t* srow, int d, double sqn,
                                     double sqd) {
    return ref_acc_q4<OP>(qf, prow, srow, d).finish(sqn, sqd);
}

// ------------------------------------------------------------ error bounds
//
// The scans rank rows by a quantized-query score (E16 codes: q^ = qs*code,
// |q - q^| = G).  For a row whose scan score is c, the reference score lies in
// [ref_lo(c), ref_hi(c)].  With u = 2^-24, |q| the query norm, |q^| its
// quantized norm, DN >= max |d'| and BB >= max |d'|^2 over the rows (d' the
// exact products code*scale, |d - d'| <= u|d'|), and e the relative error
// bound of the scan's q^.d' term (e_qd):
//   dot:    |scan - ref| <= DN (G (1 + e) + |q| (e + u + 1.01 gamma_D)) + D 2^-149
//           (gamma_D = D u / (1 - D u) bounds the f32 sequential sum)
//   cosine: |scan - ref| <= 2 G/|q| + e + 7.1 u + 2^-40
//           (|u/|u| - v/|v|| <= 2|u - v|/|u| for the query and the row; the
//           scan's division and norms add 4.1 u, the reference's narrowing u)
//   l2:     the scan's dist^2 is within Dl = (5u + e) 1.02 (|q^|^2 + BB) of
//           |q^ - d'|^2; |q - d| is within G' = G + u DN of |q^ - d'|; the
//           reference is |q - d| (1 +- 2.1 u).
// Each bound is widened by a relative 2^-40 for its own f64 evaluation.
struct RefBounds {
    double m;     // dot / cosine: absolute margin
    double gp;    // l2: G'
    double dl;    // l2: Dl
    int op;
    bool ok;      // every quantity finite
};

__device__ inline RefBounds ref_bounds(int op, double G, double qn, double qh, double e_qd, double DN, double BB,
                                       int d) {
    const double u = 5.9604644775390625e-08;
    const double up = 1.0 + 9.094947017729282e-13;  // 1 + 2^-40
    RefBounds b;
    b.op = op;
    b.m = 0.0;
    b.gp = 0.0;
    b.dl = 0.0;
    if (op == OP_DOT) {
        const double gam = (double)d * u / (1.0 - (double)d * u);
        b.m = (DN * (G * (1.0 + e_qd) + qn * (e_qd + u + 1.01 * gam)) + (double)d * 1.401298464324817e-45) * up;
    } else if (op == OP_COSINE) {
        b.m = (qn > 0.0 ? 2.0 * G / qn : 0.0) + e_qd + 7.1 * u + 9.094947017729282e-13;
        b.m *= up;
    } else {
        b.gp = (G + u * DN) * up;
        b.dl = (5.0 * u + e_qd) * 1.02 * (qh * qh + BB) * up;
    }
    b.ok = __builtin_isfinite(b.m) && __builtin_isfinite(b.gp) && __builtin_isfinite(b.dl);
    return b;
}

// Largest reference score a row of scan score c can have.
__device__ inline double ref_hi(const RefBounds& b, double c) {
    const double up = 1.0 + 9.094947017729282e-13;
    if (b.op != OP_L2) return (c + b.m) * (c + b.m >= 0.0 ? up : 1.0 / up);
    const double s = c * (1.0 + 1.1920928955078125e-07);
    return (__builtin_sqrt(s * s + b.dl) + b.gp) * (1.0 + 2.1 * 5.9604644775390625e-08) * up;
}

// Smallest reference score a row of scan score c can have.
__device__ inline double ref_lo(const RefBounds& b, double c) {
    const double up = 1.0 + 9.094947017729282e-13;
    if (b.op != OP_L2) return (c - b.m) * (c - b.m >= 0.0 ? 1.0 / up : up);
    const double s = c * (1.0 - 1.1920928955078125e-07);
    const double t = s * s - b.dl;
    const double r = (t > 0.0 ? __builtin_sqrt(t) : 0.0) - b.gp;
    return r > 0.0 ? r * (1.0 - 2.1 * 5.9604644775390625e-08) / up : 0.0;
}

}  // namespace manta
