// pack.hpp -- host-side packing of f32 rows into the packed q8 / q4 candidate
// formats, and the per-row constants the bind step stores next to them.
//
// The reference keeps q4/q8 tensors as f32-backed fake-quantized values
// (runtime/backend/tensor.go:49-71, runtime/mll_export.go:858-862) with a
// per-tensor grid (runtime/embedding_trainer.go:3730-3763).  The packed
// layouts here are this library's own contract:
//   q8 rows   : int8 code = clamp(round((x*127)/maxabs(row)), -127, 127),
//               f32 scale = maxabs/127 per row.
//   q4 blocks : 32 values per block along D, code = clamp(round((x*7)/maxabs),
//               -7, 7), two's-complement nibbles, two per byte, low nibble
//               first; f16 scale = maxabs/7 per block.
// round() is half away from zero (C roundf, Go math.Round).
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>

namespace manta {

inline float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-8f;  // m * 2^-24, exact
        return sign ? -v : v;
    }
    uint32_t bits = (e == 31) ? (sign | 0x7F800000u | (m << 13))
                              : (sign | ((e + 112u) << 23) | (m << 13));
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

inline uint16_t float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) {
        float a;
        std::memcpy(&a, &ax, 4);
        return (uint16_t)(sign | (uint32_t)std::nearbyint(a * 16777216.0f));
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7FFFFFu) >> 13);
    uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

// One q8 row: d values -> d codes (written at dst) and its scale.
inline float pack_q8_row(const float* x, int64_t d, int8_t* dst) {
    float maxabs = 0.0f;
    for (int64_t c = 0; c < d; c++) maxabs = std::fmax(maxabs, std::fabs(x[c]));
    if (maxabs == 0.0f) {
        std::memset(dst, 0, (size_t)d);
        return 0.0f;
    }
    for (int64_t c = 0; c < d; c++) {
        float v = (x[c] * 127.0f) / maxabs;
        float q = std::round(v);
        q = q > 127.0f ? 127.0f : (q < -127.0f ? -127.0f : q);
        dst[c] = (int8_t)q;
    }
    return maxabs / 127.0f;
}

// One q4 row (d % 32 == 0): d/2 packed bytes and d/32 f16 scales.
inline void pack_q4_row(const float* x, int64_t d, uint8_t* dst, uint16_t* scales) {
    for (int64_t b = 0; b < d / 32; b++) {
        const float* blk = x + b * 32;
        float maxabs = 0.0f;
        for (int c = 0; c < 32; c++) maxabs = std::fmax(maxabs, std::fabs(blk[c]));
        for (int j = 0; j < 16; j++) {
            int code[2] = {0, 0};
            for (int h = 0; h < 2; h++) {
                if (maxabs == 0.0f) continue;
                float v = (blk[2 * j + h] * 7.0f) / maxabs;
                float q = std::round(v);
                q = q > 7.0f ? 7.0f : (q < -7.0f ? -7.0f : q);
                code[h] = (int)q;
            }
            dst[b * 16 + j] = (uint8_t)((code[0] & 0xF) | ((code[1] & 0xF) << 4));
        }
        scales[b] = float_to_half(maxabs == 0.0f ? 0.0f : maxabs / 7.0f);
    }
}

// ---- exact repacking of symmetric grids
//
// The reference's fake quantization stores v' = fl32(q * scale) with q an
// integer in [-levels, levels] and scale = fl32(maxabs / levels)
// (fakeQuantizeDataInPlace, runtime/embedding_trainer.go:3738-3763).  Values
// on such a grid repack exactly: codes q with f32 scale `scale` reproduce
// every value as the f32 product code*scale (-0 becomes code 0, whose
// product +0 compares equal and adds identically in every score).

// Codes of x[0..count) on the grid of step s, or false if some value is not
// fl32(q*s) for an integer |q| <= levels.
inline bool grid_codes(const float* x, int64_t count, float s, int levels, int8_t* codes) {
    if (!(s >= 0.0f) || !std::isfinite(s)) return false;
    for (int64_t i = 0; i < count; i++) {
        const float v = x[i];
        if (s == 0.0f) {
            if (v != 0.0f) return false;
            codes[i] = 0;
            continue;
        }
        const float q = std::round(v / s);
        if (!(std::fabs(q) <= (float)levels)) return false;
        if ((float)q * s != v) return false;
        codes[i] = (int8_t)q;
    }
    return true;
}

// The grid of x[0..count) as the reference would have built it: the step
// fl32(maxabs / levels) of the grid's own maximum, or (when rounding moved
// the maximum by an ulp) one of its neighbouring f32 values.  Returns the
// step, or -1 if no candidate reproduces every value.
inline float grid_scale(const float* x, int64_t count, int levels, int8_t* codes) {
    float maxabs = 0.0f;
    for (int64_t i = 0; i < count; i++) {
        if (!std::isfinite(x[i])) return -1.0f;
        maxabs = std::fmax(maxabs, std::fabs(x[i]));
    }
    if (maxabs == 0.0f) {
        std::memset(codes, 0, (size_t)count);
        return 0.0f;
    }
    const float s0 = maxabs / (float)levels;
    const float cand[5] = {s0, std::nextafter(s0, 0.0f), std::nextafter(s0, 2.0f * s0),
                           std::nextafter(std::nextafter(s0, 0.0f), 0.0f),
                           std::nextafter(std::nextafter(s0, 2.0f * s0), 2.0f * s0)};
    for (float s : cand)
        if (s > 0.0f && grid_codes(x, count, s, levels, codes)) return s;
    return -1.0f;
}

inline int q4_nibble(const uint8_t* row, int64_t c) {
    int v = (c & 1) ? (row[c >> 1] >> 4) : (row[c >> 1] & 0xF);
    return v >= 8 ? v - 16 : v;
}

// Per-row constants of the dequantized row: |row| and |row|^2, computed in
// f64 and narrowed once.
inline void q8_row_consts(const int8_t* codes, float scale, int64_t d, float* dnorm, float* dd) {
    int64_t ss = 0;
    for (int64_t c = 0; c < d; c++) ss += (int64_t)codes[c] * codes[c];
    double s = (double)scale;
    *dnorm = (float)(std::sqrt((double)ss) * s);
    *dd = (float)((double)ss * s * s);
}

// The reference's per-row norm term of cosineRows (tensor_ops.go:1411-1421):
// sqrt of the f64 sum, in column order, of the squared f32 values the row
// stands for (q8: code*scale in f32; q4: code*f16scale, exact).  Each square
// is exact in f64.
inline double q8_row_ref_norm(const int8_t* codes, float scale, int64_t d) {
    double s = 0.0;
    for (int64_t c = 0; c < d; c++) {
        const double v = (double)((float)codes[c] * scale);
        s = s + v * v;
    }
    return std::sqrt(s);
}

inline double q4_row_ref_norm(const uint8_t* row, const uint16_t* scales, int64_t d) {
    double s = 0.0;
    for (int64_t c = 0; c < d; c++) {
        const double v = (double)((float)q4_nibble(row, c) * half_to_float(scales[c / 32]));
        s = s + v * v;
    }
    return std::sqrt(s);
}

inline void q4_row_consts(const uint8_t* row, const uint16_t* scales, int64_t d, float* dnorm,
                          float* dd) {
    double acc = 0.0;
    for (int64_t b = 0; b < d / 32; b++) {
        int64_t ss = 0;
        for (int64_t c = b * 32; c < b * 32 + 32; c++) {
            int64_t v = q4_nibble(row, c);
            ss += v * v;
        }
        double s = (double)half_to_float(scales[b]);
        acc += (s * s) * (double)ss;
    }
    *dd = (float)acc;
    *dnorm = (float)std::sqrt(acc);
}

}  // namespace manta
