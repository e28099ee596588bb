// device_common.hpp -- device helpers shared by the gfx950 kernels.
//
//  * exact f32 arithmetic for the scoring epilogues (every op rounded on its
//    own, no contraction), so GPU scores equal the CPU contract bit for bit;
//  * 64-bit selection keys giving topKTensor's total order
//    (runtime/backend/tensor_ops.go:1539-1551: value desc, index asc);
//  * a workgroup-wide top-k reservoir in LDS (threshold filter + bitonic
//    compaction) used by the fused scoring kernels and by the merge pass.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma clang fp contract(off)

namespace manta {

typedef int v4i __attribute__((ext_vector_type(4)));

struct QConst {
    float a;  // e8: qmax      e16: qs
    float b;  // e16: |q|
    float c;  // e16: |q|^2
    float d;
};

__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// C roundf: half away from zero.  x - trunc(x) is exact for every finite x.
__device__ __forceinline__ float round_half_away(float x) {
    float t = __builtin_truncf(x);
    float d = x - t;
    if (__builtin_fabsf(d) >= 0.5f) t += __builtin_copysignf(1.0f, x);
    return t;
}

// Inclusive prefix sum over the 64 lanes of a wave (all lanes active): DPP
// row shifts by 1, 2, 4 and 8 sum within each 16-lane row, then lane 15's
// total is added to rows 1 and 3 and lane 31's to rows 2 and 3.  Lanes whose
// shift source lies outside their row add 0.
__device__ __forceinline__ int wave_incl_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);   // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);   // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);   // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);   // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
    return x;
}

// Every operation rounded on its own.  Written as plain operators under this
// file's `fp contract(off)`: HIP's __fmul_rn / __fadd_rn are plain operators
// in headers compiled with contraction allowed, so a product from them fed
// into a sum may be fused into one fma (found by the reference l2 parity
// test: q - code*scale computed exactly instead of after the product's
// rounding).
__device__ __forceinline__ float fmul_rn(float a, float b) { return a * b; }
__device__ __forceinline__ float fadd_rn(float a, float b) { return a + b; }
__device__ __forceinline__ float fsub_rn(float a, float b) { return a - b; }
__device__ __forceinline__ double dmul_rn(double a, double b) { return a * b; }
__device__ __forceinline__ float fdiv_rn(float a, float b) { return __fdiv_rn(a, b); }
// __fsqrt_rn lowers to the bare v_sqrt_f32 (about 1 ulp); llvm.sqrt.f32 with
// -fhip-fp32-correctly-rounded-divide-sqrt is the correctly rounded sequence.
__device__ __forceinline__ float fsqrt_rn(float a) { return __builtin_sqrtf(a); }

// geluTensor: 0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3))), f32 with the
// tanh in f64.
__device__ __forceinline__ float gelu_value(float v) {
    const float cubic = fmul_rn(fmul_rn(v, v), v);
    const float inner = fmul_rn(0.7978845608f, fadd_rn(v, fmul_rn(0.044715f, cubic)));
    return fmul_rn(fmul_rn(0.5f, v), fadd_rn(1.0f, (float)tanh((double)inner)));
}
// The same formula with the tanh in f32 (the device library's tanhf): for the
// encoder's f16 weight GEMMs, whose operands are rounded to f16 anyway, so the
// f64 tanh buys nothing there and costs most of the FFN up-projection.
__device__ __forceinline__ float gelu_value_f32(float v) {
    const float cubic = fmul_rn(fmul_rn(v, v), v);
    const float inner = fmul_rn(0.7978845608f, fadd_rn(v, fmul_rn(0.044715f, cubic)));
    return fmul_rn(fmul_rn(0.5f, v), fadd_rn(1.0f, tanhf(inner)));
}

// Records an out-of-range gather index.  The reference's gather loops stop
// at the first bad index in position order (tensor_ops.go:751-979), so the
// lowest position must win however the threads race: the word holds
// ~(pos << 32 | index) and keeps the largest such value (0 = none; pos <
// 2^31 keeps every recorded word non-zero).  gather_error_index decodes it.
__device__ __forceinline__ void report_gather_error(unsigned long long* err, int64_t pos, int idx) {
    if (err) atomicMax(err, ~(((unsigned long long)pos << 32) | (unsigned long long)(uint32_t)idx));
}

// ----------------------------------------------------------- query codes

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


// Order-preserving map float -> u32 with -0 folded onto +0 (the reference
// compares with <, >, so -0 and +0 tie and fall through to the index).
__device__ __forceinline__ uint32_t float_order(float s) {
    uint32_t b = __float_as_uint(s);
    if (b == 0x80000000u) b = 0u;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float order_float(uint32_t o) {
    uint32_t b = (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o;
    return __uint_as_float(b);
}

// Larger key == better.  Valid keys are never 0 (the low word ~idx has its
// top bit set for idx < 2^31), so 0 is the "empty" key.
__device__ __forceinline__ uint64_t make_key(float score, uint32_t idx, int smallest) {
    uint32_t o = float_order(score);
    if (smallest) o = ~o;
    return ((uint64_t)o << 32) | (uint64_t)(~idx);
}

__device__ __forceinline__ uint32_t key_index(uint64_t key) { return ~(uint32_t)key; }

__device__ __forceinline__ float key_score(uint64_t key, int smallest) {
    uint32_t o = (uint32_t)(key >> 32);
    if (smallest) o = ~o;
    return order_float(o);
}

// ---------------------------------------------------------------- top-k

// LDS state of a block reservoir: keys[cap] (cap a power of two), count and
// threshold.  Invariant between rounds: keys[0..cnt) are distinct offered
// keys; if cnt == k after a compaction they are the k best seen so far and
// tau is the k-th, otherwise tau == 0 and nothing was dropped.
struct TopKShared {
    int cnt;
    int pad;
    uint64_t tau;
};

__device__ __forceinline__ int next_pow2(int x) {
    int p = 2;
    while (p < x) p <<= 1;
    return p;
}

// Bitonic sort, descending, of keys[0..S) (S a power of two) by the whole
// workgroup.  Ends with a barrier.
__device__ inline void block_sort_desc(uint64_t* keys, int S) {
    const int tid = threadIdx.x;
    const int nt = blockDim.x;
    for (int size = 2; size <= S; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < (S >> 1); i += nt) {
                int lo = 2 * i - (i & (stride - 1));
                int hi = lo + stride;
                bool desc = (lo & size) == 0;
                uint64_t a = keys[lo];
                uint64_t b = keys[hi];
                if (desc ? (a < b) : (a > b)) {
                    keys[lo] = b;
                    keys[hi] = a;
                }
            }
            __syncthreads();
        }
    }
}

__device__ __forceinline__ void topk_init(uint64_t* keys, TopKShared* st) {
    if (threadIdx.x == 0) {
        st->cnt = 0;
        st->tau = 0;
    }
    __syncthreads();
}

// Offer one key per thread (0 = nothing).  Keys above the threshold are
// appended; one LDS atomic per wave.  Caller guarantees room for
// blockDim.x more keys, and calls block_sync afterwards.
__device__ __forceinline__ void topk_offer(uint64_t key, uint64_t tau, uint64_t* keys,
                                           TopKShared* st) {
    const int lane = threadIdx.x & 63;
    bool take = key > tau;
    uint64_t mask = __ballot(take);
    if (mask == 0) return;
    int leader = __ffsll((unsigned long long)mask) - 1;
    int base = 0;
    if (lane == leader) base = atomicAdd(&st->cnt, __popcll(mask));
    base = __shfl(base, leader);
    if (take) {
        uint64_t below = lane ? (mask & ((~0ull) >> (64 - lane))) : 0ull;
        keys[base + __popcll(below)] = key;
    }
}

constexpr int kMaxCap = 4096;  // largest reservoir (keys per thread <= kMaxCap / 256)
static_assert(kMaxCap == 4096, "reservoir bound shared with kernels.hpp");

// Scratch of the block radix select.
struct SelectShared {
    int hist[256];
    int digit;
    int above;
    int wpos;
    int pad;
    uint64_t minkey;
};

// Keep the best k of the reservoir: a radix select over the 64-bit keys
// (8-bit digits, most significant first) finds the prefix shared by the k-th
// largest key; the keys at or above it -- exactly k, keys being distinct --
// are moved to keys[0..k) in no particular order and tau becomes the
// smallest of them.  Whole workgroup (blockDim.x == 256), after a barrier.
__device__ inline void topk_compact(uint64_t* keys, TopKShared* st, int k) {
    __shared__ SelectShared ss;
    const int tid = threadIdx.x;
    const int c = st->cnt;
    if (c <= k) {
        // nothing to drop; tau stays 0 unless exactly k keys are held
        if (tid == 0) ss.minkey = ~0ull;
        __syncthreads();
        if (c == k) {
            for (int i = tid; i < c; i += 256) atomicMin(&ss.minkey, keys[i]);
        }
        __syncthreads();
        if (tid == 0) st->tau = (c == k) ? ss.minkey : 0ull;
        __syncthreads();
        return;
    }
    uint64_t prefix = 0, pmask = 0;
    int remaining = k;
    for (int shift = 56; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += 256) ss.hist[i] = 0;
        __syncthreads();
        for (int i = tid; i < c; i += 256) {
            const uint64_t key = keys[i];
            if ((key & pmask) == prefix) atomicAdd(&ss.hist[(int)((key >> shift) & 0xFF)], 1);
        }
        __syncthreads();
        if (tid < 64) {
            // lane l owns digits 255-4l .. 252-4l (descending)
            int h[4];
            int sum = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                h[j] = ss.hist[255 - 4 * tid - j];
                sum += h[j];
            }
            const int incl = wave_incl_scan(sum);
            int cum = incl - sum;  // keys with a larger digit
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (cum < remaining && cum + h[j] >= remaining) {
                    ss.digit = 255 - 4 * tid - j;
                    ss.above = cum;
                }
                cum += h[j];
            }
        }
        __syncthreads();
        const int d = ss.digit;
        remaining -= ss.above;
        prefix |= (uint64_t)d << shift;
        pmask |= 0xFFull << shift;
        const bool all_in = ss.hist[d] == remaining;
        __syncthreads();
        if (all_in) break;  // every key with this prefix is kept
    }
    // compact: keys whose masked prefix is >= prefix (exactly k of them).
    // All reads finish (barrier) before the first write.
    uint64_t v[kMaxCap / 256];
    uint32_t keep = 0;
#pragma unroll
    for (int j = 0; j < kMaxCap / 256; j++) {
        const int i = tid + 256 * j;
        v[j] = 0;
        if (i < c) {
            v[j] = keys[i];
            if ((v[j] & pmask) >= prefix) keep |= 1u << j;
        }
    }
    if (tid == 0) {
        ss.wpos = 0;
        ss.minkey = ~0ull;
    }
    __syncthreads();
    uint64_t lo = ~0ull;
#pragma unroll
    for (int j = 0; j < kMaxCap / 256; j++) {
        if (keep & (1u << j)) {
            const int pos = atomicAdd(&ss.wpos, 1);
            keys[pos] = v[j];
            lo = v[j] < lo ? v[j] : lo;
        }
    }
    if (keep) atomicMin(&ss.minkey, lo);
    __syncthreads();
    if (tid == 0) {
        st->cnt = k;
        st->tau = ss.minkey;
    }
    __syncthreads();
}

// Sort keys[0..n) descending (n <= kMaxCap), zero-padding to a power of two.
__device__ inline void topk_sort(uint64_t* keys, int n) {
    const int S = next_pow2(n < 2 ? 2 : n);
    for (int i = n + (int)threadIdx.x; i < S; i += blockDim.x) keys[i] = 0;
    __syncthreads();
    block_sort_desc(keys, S);
}

// Compact when another round of blockDim.x offers might not fit.
// The barrier after reading the count keeps every thread's decision equal:
// no thread starts the next round's appends before all have read it.
__device__ __forceinline__ void topk_maybe_compact(uint64_t* keys, TopKShared* st, int k,
                                                   int cap) {
    int c = st->cnt;
    __syncthreads();
    if (c + (int)blockDim.x > cap) topk_compact(keys, st, k);
}

// ------------------------------------------------- wave-resident top list

// For k <= 64 a wave keeps its best keys seen so far sorted across its
// lanes: lane i holds the i-th largest (0 = empty slot).  A key enters only
// if it beats the k-th entry (thr), so after the first few batches almost
// every offer is a single compare and ballot; nothing touches LDS and no
// barrier is needed.  Keys are distinct (they carry the row index).

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int lane) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
    return ((uint64_t)hi << 32) | lo;
}

// Lane i receives lane i-1's value; lane 0 receives `first` (DPP wave_shr:1).
__device__ __forceinline__ uint64_t wave_shr1_u64(uint64_t v, uint64_t first) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)first, (int)(uint32_t)v, 0x138,
                                                               0xf, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)(first >> 32),
                                                               (int)(uint32_t)(v >> 32), 0x138, 0xf, 0xf, false);
    return ((uint64_t)hi << 32) | lo;
}

// Insert the wave-uniform key x (not already present) into the sorted list:
// lanes holding larger keys keep them, the first lane below x takes x, the
// rest shift down one lane (the last entry drops off).
__device__ __forceinline__ void wave_list_insert(uint64_t& list, uint64_t x) {
    const uint64_t prev = wave_shr1_u64(list, ~0ull);
    const bool keep = list > x;
    list = keep ? list : (prev > x ? x : prev);
}

// Offer one key per lane (0 = nothing); thr is the list's k-th entry
// (0 while fewer than k keys are held) and is kept current.
__device__ __forceinline__ void wave_list_offer(uint64_t key, uint64_t& list, uint64_t& thr, int k) {
    uint64_t mask = __ballot(key > thr);
    while (mask) {
        const int j = __ffsll((unsigned long long)mask) - 1;
        wave_list_insert(list, readlane_u64(key, j));
        thr = readlane_u64(list, k - 1);
        mask &= mask - 1;
        mask &= __ballot(key > thr);
    }
}

// The first offer to an empty list: the batch's keys take their places by
// rank (each lane counts the batch keys above its own through this wave's 64
// LDS slots, wbuf), so lane i ends holding the i-th largest with no chain of
// insertions.  The lanes trade values through wbuf: LDS operations of one
// wave run in order in the hardware, and the empty asm statements with a
// memory clobber keep the compiler from answering a read from the thread's
// own earlier store (another lane's store sits in between).
__device__ __forceinline__ void wave_list_first_fill(uint64_t key, uint64_t& list, uint64_t& thr, int k,
                                                     uint64_t* wbuf) {
    const int lane = threadIdx.x & 63;
    wbuf[lane] = key;
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
    int rank = 0;
    if (key)
        for (int j = 0; j < 64; j++) rank += wbuf[j] > key ? 1 : 0;
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
    wbuf[lane] = 0ull;
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
    if (key) wbuf[rank] = key;  // keys are distinct: so are their ranks
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
    list = wbuf[lane];
    thr = readlane_u64(list, k - 1);
}

// Merge the lists of all waves of the workgroup into wave 0's (whole
// workgroup; buf holds blockDim.x keys of LDS, at least the waves' k each).
// By rank: the waves' k entries go to buf side by side, each held key
// counts the held keys above it (LDS broadcast reads, no dependent steps),
// and the k best land at their ranks, already sorted (C0: 81.1 -> 80.7 us a
// 32-problem launch, one query's call 15.76 -> 15.26 us, against inserting
// the other waves' keys into wave 0's list one at a time).  Ends with a
// barrier.
__device__ inline void wave_lists_merge(uint64_t& list, uint64_t& thr, int k, uint64_t* buf) {
    __shared__ uint64_t wres[64];  // k <= 64 on the list path
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = (int)(blockDim.x >> 6) * k;
    if (lane < k) buf[wave * k + lane] = list;
    if (threadIdx.x < 64) wres[threadIdx.x] = 0ull;
    __syncthreads();
    const int t = (int)threadIdx.x;
    const uint64_t mine = t < n ? buf[t] : 0ull;
    int rank = 0;
    if (mine)
        for (int j = 0; j < n; j++) rank += buf[j] > mine ? 1 : 0;
    if (mine && rank < k) wres[rank] = mine;  // keys are distinct: so are their ranks
    __syncthreads();
    if (wave == 0) {
        list = lane < k ? wres[lane] : 0ull;
        thr = readlane_u64(list, k - 1);
    }
    __syncthreads();
}

}  // namespace manta
