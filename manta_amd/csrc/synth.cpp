// synth.cpp -- deterministic synthetic workloads for the retrieval hot path.
//
// The reference has no generator for these shapes, so the stream is defined
// here:  u64(seed, tensor, i) = splitmix64(key(seed, tensor) + i), uniform
// doubles from the top 53 bits, normals by Box-Muller over element pairs
// (2j, 2j+1): r = sqrt(-2 ln(1-u0)), z = r*cos(2*pi*u1) (even) or
// r*sin(2*pi*u1) (odd).  Rows are generated in f64, optionally L2-normalized
// in f64, narrowed to f32 and then either rounded to f16 or packed with the
// library's q8/q4 packers (pack.hpp).  Every element depends only on
// (seed, tensor, index), so generation is parallel and chunkable.
#include <cmath>
#include <cstdint>
#include <vector>

#include "pack.hpp"

namespace {

inline uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t stream_key(uint64_t seed, uint64_t tensor) {
    return splitmix64(splitmix64(seed ^ 0x6D616E7461ull) + tensor * 0xD1B54A32D192ED03ull);
}

inline double uniform(uint64_t key, uint64_t i) {
    return (double)(splitmix64(key + i) >> 11) * (1.0 / 9007199254740992.0);
}

inline double normal(uint64_t key, uint64_t i) {
    uint64_t j = i >> 1;
    double u0 = uniform(key, 2 * j);
    double u1 = uniform(key, 2 * j + 1);
    double r = std::sqrt(-2.0 * std::log(1.0 - u0));
    double a = 6.283185307179586 * u1;
    return (i & 1) ? r * std::sin(a) : r * std::cos(a);
}

// Row r of an [n, d] N(0,1) tensor, optionally L2-normalized, as f32.
void normal_row(uint64_t key, int64_t r, int64_t d, int normalize, double sigma, float* out,
                std::vector<double>& tmp) {
    tmp.resize((size_t)d);
    double ss = 0.0;
    for (int64_t c = 0; c < d; c++) {
        double z = normal(key, (uint64_t)(r * d + c));
        tmp[(size_t)c] = z;
        ss += z * z;
    }
    double inv = 1.0;
    if (normalize && ss > 0.0) inv = 1.0 / std::sqrt(ss);
    for (int64_t c = 0; c < d; c++) {
        double v = normalize ? tmp[(size_t)c] * inv : tmp[(size_t)c];
        out[c] = (float)(v * sigma);
    }
}

}  // namespace

extern "C" {

void manta_synth_normal_rows_f32(uint64_t seed, uint64_t tensor, int64_t n, int64_t d,
                                 double sigma, int normalize, float* out) {
    uint64_t key = stream_key(seed, tensor);
#pragma omp parallel
    {
        std::vector<double> tmp;
#pragma omp for schedule(static)
        for (int64_t r = 0; r < n; r++) normal_row(key, r, d, normalize, sigma, out + r * d, tmp);
    }
}

void manta_synth_normal_rows_f16(uint64_t seed, uint64_t tensor, int64_t n, int64_t d,
                                 double sigma, int normalize, uint16_t* out) {
    uint64_t key = stream_key(seed, tensor);
#pragma omp parallel
    {
        std::vector<double> tmp;
        std::vector<float> row((size_t)d);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < n; r++) {
            normal_row(key, r, d, normalize, sigma, row.data(), tmp);
            for (int64_t c = 0; c < d; c++) out[r * d + c] = manta::float_to_half(row[(size_t)c]);
        }
    }
}

// q8 rows, packed with the library's packer; rows are N(0,1), optionally
// L2-normalized before quantization.
void manta_synth_q8_rows(uint64_t seed, uint64_t tensor, int64_t n, int64_t d, int normalize,
                         int8_t* codes, float* scales) {
    uint64_t key = stream_key(seed, tensor);
#pragma omp parallel
    {
        std::vector<double> tmp;
        std::vector<float> row((size_t)d);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < n; r++) {
            normal_row(key, r, d, normalize, 1.0, row.data(), tmp);
            scales[r] = manta::pack_q8_row(row.data(), d, codes + r * d);
        }
    }
}

void manta_synth_q4_rows(uint64_t seed, uint64_t tensor, int64_t n, int64_t d, int normalize,
                         uint8_t* packed, uint16_t* scales) {
    uint64_t key = stream_key(seed, tensor);
#pragma omp parallel
    {
        std::vector<double> tmp;
        std::vector<float> row((size_t)d);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < n; r++) {
            normal_row(key, r, d, normalize, 1.0, row.data(), tmp);
            manta::pack_q4_row(row.data(), d, packed + r * (d / 2), scales + r * (d / 32));
        }
    }
}

// Uniform integers in [lo, hi): lo + floor(u * (hi - lo)).
void manta_synth_uniform_i32(uint64_t seed, uint64_t tensor, int64_t n, int32_t lo, int32_t hi,
                             int32_t* out) {
    uint64_t key = stream_key(seed, tensor);
    double span = (double)hi - (double)lo;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        int64_t v = (int64_t)lo + (int64_t)std::floor(uniform(key, (uint64_t)i) * span);
        if (v >= hi) v = hi - 1;
        out[i] = (int32_t)v;
    }
}

// Uniform int8 codes in [lo, hi] (inclusive), e.g. a q8 projection.
void manta_synth_uniform_i8(uint64_t seed, uint64_t tensor, int64_t n, int32_t lo, int32_t hi,
                            int8_t* out) {
    uint64_t key = stream_key(seed, tensor);
    double span = (double)hi - (double)lo + 1.0;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        int64_t v = (int64_t)lo + (int64_t)std::floor(uniform(key, (uint64_t)i) * span);
        if (v > hi) v = hi;
        out[i] = (int8_t)v;
    }
}

}  // extern "C"
