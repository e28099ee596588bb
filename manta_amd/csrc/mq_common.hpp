// mq_common.hpp -- device helpers shared by the multi-query kernels
// (kernels_mq.hip: q8 rows, kernels_mq4.hip: q4 blocks) and their select.
#pragma once

#include "device_common.hpp"
#include "kernels.hpp"

namespace manta {

typedef int v16i __attribute__((ext_vector_type(16)));

enum { MQ_E8 = 0, MQ_E16 = 1 };
enum { MQ_SCORES = 0, MQ_APPEND = 1 };

// Conservative pre-score bounds from a threshold key.  Survivors of the
// bound are re-checked with the exact key, so the bound only has to be
// loose on the safe side (relative 2^-20 covers every rounding in the
// pre-scores and in the exact score formulas).
__device__ __forceinline__ float loosen_down(float x) {
    return x - __builtin_fabsf(x) * 9.5367431640625e-7f - 1e-30f;
}
__device__ __forceinline__ float loosen_up(float x) {
    return x + __builtin_fabsf(x) * 9.5367431640625e-7f + 1e-30f;
}

// Pre-score bound of one query from its threshold key.  dot compares s*acc
// against (tau*127)/qmax; dot16 compares qd against tau; l2 compares dist^2
// against tau^2; cosine compares
// q.d against (tau*|q|) * |d| (the |d| factor is applied per row).  No
// threshold lets everything through.
template <int OP>
__device__ __forceinline__ float mq_bound(uint64_t tk, const QConst& qc, bool smallest) {
    const float open = smallest ? __builtin_inff() : -__builtin_inff();
    if (!tk) return open;
    const float ts = key_score(tk, smallest);
    if (OP == OP_DOT) {
        const float tt = fdiv_rn(fmul_rn(ts, 127.0f), qc.a);
        return smallest ? loosen_up(tt) : loosen_down(tt);
    }
    if (OP == OP_DOT16) return smallest ? loosen_up(ts) : loosen_down(ts);
    if (OP == OP_L2) {
        const float t2 = fmul_rn(ts, ts);
        return smallest ? loosen_up(t2) : loosen_down(t2);
    }
    return fmul_rn(smallest ? loosen_up(ts) : loosen_down(ts), qc.b);
}

// q8 dot regions of the 512-query kernel hold (bits of p) << 32 | row with
// p = fmul_rn(scale, acc); the key is the scalar dot epilogue's score.
__device__ __forceinline__ uint64_t dot_pair(float p, uint32_t row) {
    return ((uint64_t)__float_as_uint(p) << 32) | row;
}
__device__ __forceinline__ uint64_t dot_pair_key(uint64_t e, float qmax, bool smallest) {
    const float p = __uint_as_float((uint32_t)(e >> 32));
    return make_key(fdiv_rn(fmul_rn(p, qmax), 127.0f), (uint32_t)e, smallest);
}

// Direct global->LDS loads (gfx950): each lane's 16 (or 4) bytes land at
// M0 + 16*lane (4*lane) of the wave's LDS segment.  Issued from inline asm so
// the compiler does not wait for them around LDS reads of other tiles; the
// scan waits for them itself (s_waitcnt vmcnt, loads complete in order).
// The compiler's own waits stay correct: they only ever count too few
// outstanding loads and so wait longer, never shorter.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p);
}
__device__ __forceinline__ void lds_load16(const void* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void lds_load4(const void* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}

// Scratch of block_radix_prefix: histograms and results double-buffered by
// round, so a round needs only two barriers.
struct RadixShared {
    int hist[2][256];
    int digit[2];
    int above[2];
    int count[2];
};

// Radix select over keys[0..c) (c > k, keys distinct), whole workgroup:
// finds (prefix, pmask) such that exactly k keys satisfy
// (key & pmask) >= prefix.  8-bit digits, most significant first; a wave
// whose matching lanes share one digit adds them with a single LDS atomic,
// so the (typically uniform) leading digits of the keys cost no contention.
// Per round: histogram, barrier, wave 0 scans (and clears the histogram for
// the round after next), barrier, every thread reads the result.
__device__ inline void block_radix_prefix(const uint64_t* keys, int c, int k, RadixShared& rs,
                                          uint64_t& prefix_out, uint64_t& pmask_out) {
    const int tid = threadIdx.x;
    const int nt = blockDim.x;
    const int lane = tid & 63;
    for (int i = tid; i < 512; i += nt) (&rs.hist[0][0])[i] = 0;
    __syncthreads();
    uint64_t prefix = 0, pmask = 0;
    int remaining = k;
    int b = 0;
    for (int shift = 56; shift >= 0; shift -= 8, b ^= 1) {
        int* hist = rs.hist[b];
        for (int i = tid; i < c; i += nt) {
            const uint64_t key = keys[i];
            const bool m = (key & pmask) == prefix;
            const int dg = (int)((key >> shift) & 0xFF);
            const uint64_t mm = __ballot(m);
            if (mm) {
                const int lead = __ffsll((unsigned long long)mm) - 1;
                const int d0 = __shfl(dg, lead);
                const uint64_t same = __ballot(m && dg == d0);
                if (same == mm) {
                    if (lane == lead) atomicAdd(&hist[d0], __popcll(mm));
                } else if (m) {
                    atomicAdd(&hist[dg], 1);
                }
            }
        }
        __syncthreads();
        if (tid < 64) {
            // lane l owns digits 255-4l .. 252-4l (descending)
            int h[4];
            int sum = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                h[j] = hist[255 - 4 * tid - j];
                hist[255 - 4 * tid - j] = 0;  // ready for the round after next
                sum += h[j];
            }
            const int incl = wave_incl_scan(sum);
            int cum = incl - sum;  // keys with a larger digit
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (cum < remaining && cum + h[j] >= remaining) {
                    rs.digit[b] = 255 - 4 * tid - j;
                    rs.above[b] = cum;
                    rs.count[b] = h[j];
                }
                cum += h[j];
            }
        }
        __syncthreads();
        const int d = rs.digit[b];
        remaining -= rs.above[b];
        prefix |= (uint64_t)d << shift;
        pmask |= 0xFFull << shift;
        if (rs.count[b] == remaining) break;  // every key with this prefix is kept
    }
    prefix_out = prefix;
    pmask_out = pmask;
}

// Offset of this thread's `cnt` items in a block-wide append through
// `counter`: a wave prefix sum and one LDS atomic per wave.
__device__ __forceinline__ int wave_append(int cnt, int* counter) {
    const int lane = threadIdx.x & 63;
    const int incl = wave_incl_scan(cnt);
    int base = 0;
    if (lane == 63 && incl) base = atomicAdd(counter, incl);
    base = __shfl(base, 63);
    return base + incl - cnt;
}

// Sort keys[0..S) descending in place, whole workgroup of NT threads, with
// J = S / NT slots per thread known at compile time (S a power of two,
// NT / 2 < S <= J * NT when J > 1).  Bitonic network over registers: thread
// t holds elements t + j*NT; exchanges at strides below 64 are lane
// shuffles, at strides of NT and more stay inside a thread, and only the
// strides in between go through LDS (two barriers each).  J must be a
// constant: with a run-time slot count the slot loops stay rolled and every
// step indexes the register array dynamically.
template <int NT, int J>
__device__ __forceinline__ void block_sort_desc_regs_j(uint64_t* keys, int S) {
    const int tid = threadIdx.x;
    uint64_t v[J];
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int i = tid + j * NT;
        v[j] = i < S ? keys[i] : 0ull;
    }
    auto pick = [](uint64_t mine, uint64_t other, bool desc, bool lower) {
        const uint64_t hi = mine > other ? mine : other, lo = mine > other ? other : mine;
        return desc == lower ? hi : lo;
    };
    for (int size = 2; size <= S; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            if (stride >= NT) {
#pragma unroll
                for (int sj = 1; sj < J; sj <<= 1) {
                    if (stride != sj * NT) continue;
#pragma unroll
                    for (int j = 0; j < J; j++) {
                        if (j & sj) continue;
                        const int jp = j | sj;
                        const bool desc = ((tid + j * NT) & size) == 0;
                        const uint64_t a = v[j], c = v[jp];
                        v[j] = pick(a, c, desc, true);
                        v[jp] = pick(c, a, desc, false);
                    }
                }
            } else if (stride >= 64) {
#pragma unroll
                for (int j = 0; j < J; j++)
                    if (tid + j * NT < S) keys[tid + j * NT] = v[j];
                __syncthreads();
#pragma unroll
                for (int j = 0; j < J; j++) {
                    const int i = tid + j * NT;
                    if (i < S) v[j] = pick(v[j], keys[i ^ stride], (i & size) == 0, (i & stride) == 0);
                }
                __syncthreads();
            } else {
#pragma unroll
                for (int j = 0; j < J; j++) {
                    const int i = tid + j * NT;
                    const uint64_t other = __shfl_xor(v[j], stride);
                    if (i < S) v[j] = pick(v[j], other, (i & size) == 0, (i & stride) == 0);
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < J; j++)
        if (tid + j * NT < S) keys[tid + j * NT] = v[j];
    __syncthreads();
}

// Sort keys[0..S) descending in place (S a power of two, S <= NT*16).
template <int NT>
__device__ __forceinline__ void block_sort_desc_regs(uint64_t* keys, int S) {
    if (S <= NT) block_sort_desc_regs_j<NT, 1>(keys, S);
    else if (S <= 2 * NT) block_sort_desc_regs_j<NT, 2>(keys, S);
    else if (S <= 4 * NT) block_sort_desc_regs_j<NT, 4>(keys, S);
    else if (S <= 8 * NT) block_sort_desc_regs_j<NT, 8>(keys, S);
    else block_sort_desc_regs_j<NT, 16>(keys, S);
}

// Chunk tiles per workgroup: as many (2..4) as fit in about 72 KB of LDS
// (two workgroups per CU), and at most as many as s_waitcnt can count.
static constexpr int mq_nbuf(int tile_and_consts, int loads_per_chunk) {
    int n = 73728 / tile_and_consts;
    n = n > 4 ? 4 : n;
    while (n > 2 && (n - 2) * loads_per_chunk > 63) n--;
    return n < 2 ? 2 : n;
}

// s_waitcnt vmcnt(J*VPW) + s_barrier when at least J chunks were issued after
// the current one, else the next smaller J (a smaller count waits longer,
// never shorter).
template <int VPW, int J>
__device__ __forceinline__ void mq_wait_barrier(int64_t after) {
    if constexpr (J <= 0) {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    } else {
        if (after >= J)
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(J * VPW) : "memory");
        else
            mq_wait_barrier<VPW, J - 1>(after);
    }
}

}  // namespace manta
