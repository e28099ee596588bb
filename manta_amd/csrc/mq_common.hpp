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
// against (tau*127)/qmax; l2 compares dist^2 against tau^2; cosine compares
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
    if (OP == OP_L2) {
        const float t2 = fmul_rn(ts, ts);
        return smallest ? loosen_up(t2) : loosen_down(t2);
    }
    return fmul_rn(smallest ? loosen_up(ts) : loosen_down(ts), qc.b);
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

// Radix select over keys[0..c) (c > k, keys distinct), whole workgroup:
// finds (prefix, pmask) such that exactly k keys satisfy
// (key & pmask) >= prefix.  8-bit digits, most significant first; a wave
// whose matching lanes share one digit adds them with a single LDS atomic,
// so the (typically uniform) leading digits of the keys cost no contention.
__device__ inline void block_radix_prefix(const uint64_t* keys, int c, int k, SelectShared& ss,
                                          uint64_t& prefix_out, uint64_t& pmask_out) {
    const int tid = threadIdx.x;
    const int nt = blockDim.x;
    const int lane = tid & 63;
    uint64_t prefix = 0, pmask = 0;
    int remaining = k;
    for (int shift = 56; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += nt) ss.hist[i] = 0;
        __syncthreads();
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
                    if (lane == lead) atomicAdd(&ss.hist[d0], __popcll(mm));
                } else if (m) {
                    atomicAdd(&ss.hist[dg], 1);
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
                h[j] = ss.hist[255 - 4 * tid - j];
                sum += h[j];
            }
            int incl = sum;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const int t = __shfl_up(incl, off);
                if (tid >= off) incl += t;
            }
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
    prefix_out = prefix;
    pmask_out = pmask;
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
