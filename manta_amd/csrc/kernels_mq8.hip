// kernels_mq8.hip -- many queries against one shared q8 matrix with dot
// scores (E8 query codes), on v_mfma_i32_16x16x64_i8.
//
// mq8_scan_kernel: workgroup = 8 waves (512 threads, one workgroup per CU),
// grid = (row ranges, groups of 512 queries).  Each wave keeps 64 queries'
// codes resident as the A operand (4 blocks of 16 queries x PITCH bytes).
// Candidate rows stream through LDS in chunks of CH rows, moved by
// direct-to-LDS loads NBUF-1 chunks ahead of their use; every wave reads all
// rows of a chunk as B fragments (16 rows x 64 bytes), so each candidate
// byte is fetched from L2 once per 512 queries.  A row pair (two 16-row
// blocks) is eight independent accumulator chains of PITCH/64 MFMAs each.
//
// 16x16 output layout: lane l holds D[4*(l/16) + r][l%16], r = 0..3, i.e.
// queries 16*qb + 4*(l/16) + r of its A blocks against row l%16 of each B
// block.  The filter is one fma per (query, row): scale*acc - bound, with
// the bound loosened past the exact test's, reduced by v_max3 over a query
// block's 8 pairs per lane; only a block with a passing lane takes the
// exact f32 test p = fmul_rn(scale, acc) against the bound.  A pair that
// passes goes to its region as (bits of p) << 32 | row: the division and the
// key are left to the select kernel, where every lane has one.  Row scales
// must be finite (the runtime routes other candidates to kernels_mq.hip).
//
// The LDS tile stores row r's 16-byte column c at column c ^ ((r >> 1) & 7)
// (PITCH is a multiple of 128, so a row holds a multiple of 8 columns): the
// 16 lanes reading one column of 16 consecutive rows hit distinct banks.
// Top-k runs in the same threshold passes as kernels_mq.hip (regions per
// (workgroup, query), compaction when a region might overflow).
#include "mq_common.hpp"

namespace manta {

namespace {
constexpr int kMq8Waves = 8;
constexpr int kMq8Threads = kMq8Waves * 64;
constexpr int kMq8QG = kMq8Waves * 64;  // queries per workgroup
constexpr int kMq8RB = 4;               // 16-row blocks per chunk
constexpr int kMq8CH = kMq8RB * 16;     // rows per chunk

// chunk tiles within 136 KB of dynamic LDS (the static arrays take ~15 KB of 160)
constexpr int mq8_nbuf(int tile) {
    int n = 136 * 1024 / tile;
    return n > 6 ? 6 : (n < 2 ? 2 : n);
}
}  // namespace

template <int KS64, bool SMALL>
__global__ __launch_bounds__(kMq8Threads) __attribute__((amdgpu_waves_per_eu(2))) void mq8_scan_kernel(MqArgs a) {
    constexpr int PITCH = KS64 * 64;
    constexpr int CH = kMq8CH;
    constexpr int TILE = CH * PITCH;                     // bytes per chunk tile
    constexpr int LPW = TILE / 1024 / kMq8Waves;         // 16-byte direct-to-LDS loads per wave per chunk
    static_assert(LPW * 1024 * kMq8Waves == TILE, "chunk tile must split evenly over the waves");
    constexpr int NBUF = mq8_nbuf(TILE);
    static_assert((NBUF - 2) * (LPW + 1) <= 63, "vmcnt range");
    constexpr int QG = kMq8QG;
    constexpr int NFW = QG / 64;

    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* tiles = smem;                               // [NBUF][TILE]
    float* cscale = (float*)(smem + NBUF * TILE);        // [NBUF][CH] row scales
    __shared__ uint64_t tau_s[QG];
    __shared__ __attribute__((aligned(16))) float bnd_s[QG];
    __shared__ __attribute__((aligned(16))) float qa_s[QG];
    __shared__ __attribute__((aligned(16))) float pre_s[QG];  // pre-filter bounds (loosened further)
    __shared__ int cnt_s[QG];
    __shared__ uint64_t flags[2][NFW];
    __shared__ RadixShared ss;
    __shared__ int wpos;
    __shared__ unsigned long long minkey;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 4, j = lane & 15;
    const int q0 = blockIdx.y * QG;
    const int lw = wave * 64;  // this wave's first workgroup-local query

    for (int i = tid; i < QG; i += kMq8Threads) {
        const int q = q0 + i;
        const bool ok = q < a.nq;
        const QConst qc = ok ? a.qconst[q] : QConst{1.0f, 0.0f, 0.0f, 0.0f};
        const uint64_t tk = ok ? a.tau[q] : 0ull;
        qa_s[i] = qc.a;
        tau_s[i] = ok ? tk : ~0ull;
        bnd_s[i] = ok ? mq_bound<OP_DOT>(tk, qc, SMALL) : (SMALL ? -__builtin_inff() : __builtin_inff());
        pre_s[i] = SMALL ? loosen_up(bnd_s[i]) : loosen_down(bnd_s[i]);
        cnt_s[i] = 0;
    }

    // A operand: 4 blocks of 16 queries, K steps of 64 bytes
    v4i av[4][KS64];
#pragma unroll
    for (int qb = 0; qb < 4; qb++) {
        const int q = q0 + lw + qb * 16 + j;
        const bool ok = q < a.nq;
        const int8_t* src = a.qc8 + (int64_t)(ok ? q : 0) * PITCH + 16 * g;
#pragma unroll
        for (int ks = 0; ks < KS64; ks++) av[qb][ks] = ok ? *(const v4i*)(src + ks * 64) : v4i{0, 0, 0, 0};
    }

    uint64_t* wreg = a.regions + (int64_t)blockIdx.x * a.nq * a.rc;
    const int64_t r0 = a.row_begin + (int64_t)blockIdx.x * a.rows_per_wg;
    int64_t r1 = r0 + a.rows_per_wg;
    if (r1 > a.row_end) r1 = a.row_end;

    // Direct-to-LDS chunk loads: lane i of load s fills tile bytes
    // [1024 s + 16 i, +16), which hold row x / PITCH, stored column
    // (x % PITCH) / 16, i.e. source column stored ^ ((row >> 1) & 7).
    // Rows past the range read the last row of the range instead.
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);
    int soff[LPW];
#pragma unroll
    for (int i = 0; i < LPW; i++) {
        const int x = (wave_s * LPW + i) * 1024 + lane * 16;
        const int row = x / PITCH;
        const int col = ((x % PITCH) / 16) ^ ((row >> 1) & 7);
        soff[i] = row * PITCH + col * 16;
    }
    const uint32_t tbase = lds_addr(tiles);
    const uint32_t sbase = lds_addr(cscale);
    auto issue_chunk = [&](int64_t c0, int buf) {
        const int8_t* base = a.codes + c0 * PITCH;
        const int left = (int)(r1 - c0 < CH ? r1 - c0 : CH);
        const int lim = left * PITCH - 16;  // last 16 bytes of the last row in range
        // the LDS destination goes to M0: keep it in a scalar register
        const uint32_t dst = __builtin_amdgcn_readfirstlane(tbase + buf * TILE + wave_s * LPW * 1024);
#pragma unroll
        for (int i = 0; i < LPW; i++) lds_load16(base + (soff[i] < lim ? soff[i] : lim), dst + i * 1024);
        // the chunk's row scales (only the exact test reads them): one more
        // 4-byte load per lane, by the last wave
        if (wave_s == kMq8Waves - 1)
            lds_load4(a.scales + c0 + (lane < left ? lane : left - 1),
                      __builtin_amdgcn_readfirstlane(sbase + buf * CH * 4));
    };
    __syncthreads();  // query state above is complete
    // retire the A-fragment loads here, not at their first use in the loop
    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int b = 0; b < NBUF - 1; b++)
        if (r0 + b * CH < r1) issue_chunk(r0 + b * CH, b);

    // pre-filter bounds of a query block's 4 queries of this lane (one LDS read)
    auto load_bq = [&](int qb, float (&b)[4]) {
        const float4 b4 = *(const float4*)&pre_s[lw + qb * 16 + 4 * g];
        b[0] = b4.x, b[1] = b4.y, b[2] = b4.z, b[3] = b4.w;
    };
    // pre-score of one (query, row): >= 0 unless the exact test must fail
    auto pre = [&](float scale, int acc, float b) {
        return SMALL ? __fmaf_rn(-scale, (float)acc, b) : __fmaf_rn(scale, (float)acc, -b);
    };

    // The pairs of one query block of a row pair that pass the exact test,
    // appended as (pre-score, row) pairs (a wave where one passed the filter).
    auto survivors = [&](const v4i (&acc)[2][4], int qb, int64_t rb0, const float (&sc)[2], const float (&bq)[4]) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int64_t row = rb0 + h * 16 + j;
            const bool valid = row < r1;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                if (!valid || !(pre(sc[h], acc[h][qb][r], bq[r]) >= 0.0f)) continue;
                const int lq = lw + qb * 16 + 4 * g + r;
                const float p = fmul_rn(sc[h], (float)acc[h][qb][r]);
                if (SMALL ? (p > bnd_s[lq]) : (p < bnd_s[lq])) continue;
                const int pos = atomicAdd(&cnt_s[lq], 1);
                wreg[(uint32_t)((q0 + lq) * a.rc + pos)] = dot_pair(p, (uint32_t)row);
            }
        }
    };

    int buf = 0, par = 0;
    for (int64_t c0 = r0; c0 < r1; c0 += CH, buf = buf == NBUF - 1 ? 0 : buf + 1, par ^= 1) {
        // Flag regions that might not take one more chunk of keys (a count
        // read before the barrier may miss up to CH keys of the chunk other
        // waves are filtering: margin of two chunks, rc >= k + 2*CH + 1).
        {
            const int i = wave * 64 + lane;
            const uint64_t m = __ballot(cnt_s[i] > a.rc - 2 * CH);
            if (lane == 0) flags[par][wave] = m;
        }
        // this wave's loads of chunk c are done once at most the loads of
        // the chunks issued after it are outstanding; the barrier extends
        // that to every wave, retires the previous chunk's reads of the tile
        // about to be refilled, and publishes the flags
        // (the last wave issues one more load per chunk: the row scales)
        if (wave == kMq8Waves - 1)
            mq_wait_barrier<LPW + 1, NBUF - 2>((r1 - c0 - 1) / CH);
        else
            mq_wait_barrier<LPW, NBUF - 2>((r1 - c0 - 1) / CH);
        const int nbuf = buf == 0 ? NBUF - 1 : buf - 1;  // tile of chunk c+NBUF-1 (free now)
        {
            bool any = false;
#pragma unroll
            for (int w = 0; w < NFW; w++) any |= flags[par][w] != 0;
            if (any) {
                // rare: compact full regions to their best k pairs (the
                // scratch tile holds the region's keys, then its pairs)
                uint64_t* skeys = (uint64_t*)(tiles + nbuf * TILE);
                uint64_t* spairs = skeys + a.rc;
                for (int lq = 0; lq < QG; lq++) {
                    if (!((flags[par][lq >> 6] >> (lq & 63)) & 1)) continue;
                    uint64_t* reg = wreg + (uint32_t)((q0 + lq) * a.rc);
                    const int c = cnt_s[lq];
                    for (int i = tid; i < c; i += kMq8Threads) {
                        const uint64_t e = reg[i];
                        spairs[i] = e;
                        skeys[i] = dot_pair_key(e, qa_s[lq], SMALL);
                    }
                    if (tid == 0) {
                        wpos = 0;
                        minkey = ~0ull;
                    }
                    __syncthreads();
                    uint64_t prefix, pmask;
                    block_radix_prefix(skeys, c, a.k, ss, prefix, pmask);
                    uint64_t lo = ~0ull;
                    for (int i = tid; i < c; i += kMq8Threads) {
                        const uint64_t key = skeys[i];
                        if ((key & pmask) >= prefix) {
                            reg[atomicAdd(&wpos, 1)] = spairs[i];
                            lo = key < lo ? key : lo;
                        }
                    }
                    if (lo != ~0ull) atomicMin(&minkey, (unsigned long long)lo);
                    __syncthreads();
                    if (tid == 0) {
                        cnt_s[lq] = a.k;
                        if (minkey > tau_s[lq]) {
                            tau_s[lq] = minkey;
                            bnd_s[lq] = mq_bound<OP_DOT>(minkey, a.qconst[q0 + lq], SMALL);
                            pre_s[lq] = SMALL ? loosen_up(bnd_s[lq]) : loosen_down(bnd_s[lq]);
                        }
                    }
                    __syncthreads();
                }
            }
        }
        if (c0 + (NBUF - 1) * CH < r1) issue_chunk(c0 + (NBUF - 1) * CH, nbuf);
        const uint8_t* tile = tiles + buf * TILE;
#pragma unroll
        for (int rp = 0; rp < kMq8RB; rp += 2) {
            // B fragments one K step ahead of their MFMAs (the scheduling
            // barrier keeps the compiler from hoisting every step's reads,
            // which would hold all 2*KS64 fragments in registers)
            auto load_b = [&](v4i (&b)[2], int ks) {
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int row = (rp + h) * 16 + j;
                    b[h] = *(const v4i*)(tile + row * PITCH + (((ks * 4 + g) ^ ((row >> 1) & 7)) * 16));
                }
            };
            v4i acc[2][4];
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int qb = 0; qb < 4; qb++) acc[h][qb] = v4i{0, 0, 0, 0};
            v4i bc[2], bn[2];
            load_b(bc, 0);
#pragma unroll
            for (int ks = 0; ks < KS64; ks++) {
                if (ks + 1 < KS64) load_b(bn, ks + 1);
#pragma unroll
                for (int qb = 0; qb < 4; qb++)
#pragma unroll
                    for (int h = 0; h < 2; h++)
                        acc[h][qb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[qb][ks], bc[h], acc[h][qb], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                bc[0] = bn[0];
                bc[1] = bn[1];
            }
            // one fma per (query, row) and a running max (v_max3) per query block
            const int64_t rb0 = c0 + rp * 16;
            const float sc[2] = {cscale[buf * CH + rp * 16 + j], cscale[buf * CH + rp * 16 + 16 + j]};
#pragma unroll
            for (int qb = 0; qb < 4; qb++) {
                float bq[4];
                load_bq(qb, bq);
                float m = -__builtin_inff();
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int r = 0; r < 4; r++) m = fmaxf(m, pre(sc[h], acc[h][qb][r], bq[r]));
                if (__ballot(m >= 0.0f)) survivors(acc, qb, rb0, sc, bq);
            }
        }
    }
    __syncthreads();
    for (int i = tid; i < QG; i += kMq8Threads)
        if (q0 + i < a.nq) a.counts[(int64_t)blockIdx.x * a.nq + q0 + i] = cnt_s[i];
}

// pitch 512 would exceed the register budget (A fragments alone take 128)
bool mq8_supported(int pitch) { return pitch == 128 || pitch == 256 || pitch == 384; }

MqShape mq8_shape(int pitch) {
    MqShape s;
    s.kind = 1;
    s.ks = pitch / 64;
    s.na = 4;
    s.wq = kMq8Waves;
    s.qg = kMq8QG;
    s.chunk = kMq8CH;
    s.tile = kMq8CH * pitch;
    s.tile_bytes = mq8_nbuf(s.tile) * (s.tile + kMq8CH * 4);  // chunk tiles + row scales
    s.threads = kMq8Threads;
    return s;
}

template <int KS64, bool SMALL>
static hipError_t launch_mq8_one(const MqArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)mq8_scan_kernel<KS64, SMALL>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL((mq8_scan_kernel<KS64, SMALL>), grid, dim3(kMq8Threads), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_mq8_scan(const MqShape& sh, const MqArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    const bool sm = a.smallest != 0;
    switch (sh.ks) {
        case 2: return sm ? launch_mq8_one<2, true>(a, grid, lds, s) : launch_mq8_one<2, false>(a, grid, lds, s);
        case 4: return sm ? launch_mq8_one<4, true>(a, grid, lds, s) : launch_mq8_one<4, false>(a, grid, lds, s);
        case 6: return sm ? launch_mq8_one<6, true>(a, grid, lds, s) : launch_mq8_one<6, false>(a, grid, lds, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace manta
