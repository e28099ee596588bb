// kernels_mq8.hip -- many queries against one shared q8 matrix with dot
// scores (E8 query codes), on v_mfma_i32_16x16x64_i8.
//
// mq8_scan_kernel: workgroup = 8 waves (512 threads, one workgroup per CU),
// grid = (row ranges, groups of 512 / WS queries).  Each wave keeps 64
// queries' codes resident as the A operand (4 blocks of 16 queries x PITCH
// bytes).  Candidate rows stream through LDS in chunks of 64*WS rows, moved
// by direct-to-LDS loads NBUF-1 chunks ahead of their use; every wave reads
// 64 rows of a chunk (two row pairs) as B fragments (16 rows x 64 bytes), so
// each candidate byte is fetched from L2 once per 512 / WS queries.  A row
// pair (two 16-row blocks) is eight independent accumulator chains of
// PITCH/64 MFMAs each.
//
// 16x16 output layout: lane l holds D[4*(l/16) + r][l%16], r = 0..3, i.e.
// queries 16*qb + 4*(l/16) + r of its A blocks against row l%16 of each B
// block.  A wave orders its 64 queries by their current bound before the
// scan (slot L of the wave holds the L-th), so a lane's 4 queries have
// nearly equal bounds, and the pre-filter takes four VALU instructions per
// lane, query block and 16-row block: the best of the lane's 4
// accumulators, converted, times the row scale, less the loosest of the 4
// bounds (loosened past the exact test's).  The filter of a row pair runs
// under the MFMAs of the wave's next pair (a chunk's second pair under the
// next chunk's first).  Only a query block with a passing lane takes the
// exact f32 test p = fmul_rn(scale, acc), against the loosest bound of the
// lane's 4 queries (or, for shadow pairs and query counts that are not a
// multiple of 4, each query's own bound: OWNB).  A
// pair that passes goes to its query's region as (bits of p) << 32 | row:
// the division and the key are left to the select kernel, where every lane
// has one.  Row scales must be finite and not negative (the runtime routes
// other candidates to kernels_mq.hip).
//
// The LDS tile stores row r's 16-byte column c at column c ^ ((r >> 1) & 7)
// (PITCH is a multiple of 128, so a row holds a multiple of 8 columns): the
// 16 lanes reading one column of 16 consecutive rows hit distinct banks.
// Top-k runs in the same threshold passes as kernels_mq.hip (regions per
// (workgroup, query), compaction when a region might overflow); the first
// pass, which has no threshold, stores every pair at its row's slot without
// tests or atomics.
#include <algorithm>

#include "mq_common.hpp"
#include "q4_common.hpp"

namespace manta {

namespace {
constexpr int kMq8Waves = 8;
constexpr int kMq8Threads = kMq8Waves * 64;
constexpr int kMq8QG = kMq8Waves * 64;  // queries per workgroup
constexpr int kMq8CH = 64;             // rows per chunk and wave group (two row pairs per wave)

// chunk tiles (with their row scales) in the LDS the static arrays leave:
// those take 24 bytes per query plus about 2.5 KB
constexpr int mq8_nbuf(int tile, int qg, int ch) {
    int n = (160 * 1024 - qg * 24 - 2560) / (tile + ch * 4);
    return n > 6 ? 6 : (n < 2 ? 2 : n);
}
}  // namespace

template <int KS64, bool SMALL, int WS, bool SHADOW, bool OWNB>
__global__ __launch_bounds__(kMq8Threads) __attribute__((amdgpu_waves_per_eu(2))) void mq8_scan_kernel(MqArgs a) {
    constexpr int PITCH = KS64 * 64;
    constexpr int CH = kMq8CH * WS;                      // rows per chunk
    constexpr int PPW = CH / 32 / WS;                    // row pairs per wave and chunk
    constexpr int TILE = CH * PITCH;                     // bytes per chunk tile
    constexpr int LPW = TILE / 1024 / kMq8Waves;         // 16-byte direct-to-LDS loads per wave per chunk
    static_assert(LPW * 1024 * kMq8Waves == TILE, "chunk tile must split evenly over the waves");
    static_assert(WS == 1 || WS == 2, "one or two wave groups");
    constexpr int QG = kMq8QG / WS;          // queries per workgroup
    constexpr int NBUF = mq8_nbuf(TILE, QG, CH);
    static_assert((NBUF - 2) * (LPW + 1) <= 63, "vmcnt range");
    constexpr int NFW = QG / 64;             // waves per query group
    static_assert(PPW == 2, "a wave's two row pairs alternate between two accumulator sets");

    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* tiles = smem;                               // [NBUF][TILE]
    float* cscale = (float*)(smem + NBUF * TILE);        // [NBUF][CH] row scales
    // query state by slot: slot lw + L of a wave holds query qmap_s[lw + L]
    __shared__ uint64_t tau_s[QG];
    __shared__ __attribute__((aligned(16))) float bnd_s[QG];
    __shared__ int qmap_s[QG];
    __shared__ float pmin_s[QG / 4];  // loosest pre-filter bound of each 4 consecutive slots
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
    const int lw = (wave % NFW) * 64;  // this wave's first workgroup-local query
    const int rw = (wave / NFW) * (CH / WS);  // this wave's first row of a chunk (PPW row pairs)

    uint64_t* wreg = a.regions + (int64_t)blockIdx.x * a.nq * a.rc;
    const int64_t r0 = a.row_begin + (int64_t)blockIdx.x * a.rows_per_wg;
    int64_t r1 = r0 + a.rows_per_wg;
    if (r1 > a.row_end) r1 = a.row_end;

    // Direct-to-LDS chunk loads: lane i of load s fills tile bytes
    // [1024 s + 16 i, +16), which hold row x / PITCH, stored column
    // (x % PITCH) / 16, i.e. source column stored ^ ((row >> 1) & 7).
    // Rows past the range read the last row of the range instead.  The
    // source offsets are recomputed per chunk (the empty asm keeps the
    // compiler from hoisting them out of the loop): held in registers they
    // get spilled, and a scratch reload's vmcnt wait would also wait for the
    // chunk loads in flight.
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);
    auto soff = [&](int i) {
        int ws = wave_s;
        asm volatile("" : "+s"(ws));
        const int x = (ws * LPW + i) * 1024 + lane * 16;
        const int row = x / PITCH;
        const int col = ((x % PITCH) / 16) ^ ((row >> 1) & 7);
        return row * PITCH + col * 16;
    };
    const uint32_t tbase = lds_addr(tiles);
    const uint32_t sbase = lds_addr(cscale);
    // the last WS waves also load the chunk's row scales (64 each)
    const int sw = wave_s - (kMq8Waves - WS);
    auto issue_chunk = [&](int64_t c0, int buf) {
        const int8_t* base = a.codes + c0 * PITCH;
        const int left = (int)(r1 - c0 < CH ? r1 - c0 : CH);
        const int lim = left * PITCH - 16;  // last 16 bytes of the last row in range
        // the LDS destination goes to M0: keep it in a scalar register
        const uint32_t dst = __builtin_amdgcn_readfirstlane(tbase + buf * TILE + wave_s * LPW * 1024);
#pragma unroll
        for (int i = 0; i < LPW; i++) {
            const int o = soff(i);
            lds_load16(base + (o < lim ? o : lim), dst + i * 1024);
        }
        if (sw >= 0) {
            int sws = sw;
            asm volatile("" : "+s"(sws));  // recomputed per chunk, as soff
            const int si = sws * 64 + lane;
            lds_load4(a.scales + c0 + (si < left ? si : left - 1),
                      __builtin_amdgcn_readfirstlane(sbase + buf * CH * 4 + sw * 256));
        }
    };
    // Lane L's query (q0 + lw + L): its threshold and bound, loaded first
    // and retired before the chunk loads go out (behind those, a few
    // megabytes of chunks per XCD, they would take microseconds); the empty
    // asm keeps the query constants' load beside tau's (the bound reads them
    // only when tau is set), so one wait covers both.
    auto bound_of = [&](int q, uint64_t& tk) {
        tk = a.tau[q];
        if (SHADOW) {
            const float m = a.qbound[2 * q], f = a.qbound[2 * q + 1];
            asm volatile("" ::"v"(m), "v"(f));
            return shadow_bound(tk, m, f, SMALL);
        }
        const QConst qc = a.qconst[q];
        asm volatile("" ::"v"(qc.a));
        return mq_bound<OP_DOT>(tk, qc, SMALL);
    };
    uint64_t my_tau = ~0ull;
    float my_bnd = SMALL ? -__builtin_inff() : __builtin_inff();
    uint32_t ord = 0xFFFFFFFFu;  // missing queries go last
    {
        const int q = q0 + lw + lane;
        if (q < a.nq) {
            my_bnd = bound_of(q, my_tau);
            const uint32_t u = __float_as_uint(my_bnd);
            ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
            ord = ord == 0xFFFFFFFFu ? 0xFFFFFFFEu : ord;
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    // then the first chunks' loads; the sort and the A fragments run under them
#pragma unroll
    for (int b = 0; b < NBUF - 1; b++)
        if (r0 + b * CH < r1) issue_chunk(r0 + b * CH, b);

    // Each wave orders its 64 queries by their bound (a bitonic sort across
    // the lanes): slot lw + L takes the L-th, so the 4 queries a lane filters
    // together have nearly equal bounds.  Both wave groups of WS = 2 sort the
    // same queries the same way.
    uint64_t skey;
    {
        skey = ((uint64_t)ord << 32) | (uint32_t)lane;
#pragma unroll
        for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
            for (int jj = k >> 1; jj > 0; jj >>= 1) {
                const uint64_t o = ((uint64_t)(uint32_t)__shfl_xor((int)(skey >> 32), jj) << 32) |
                                   (uint32_t)__shfl_xor((int)(uint32_t)skey, jj);
                const bool keep_min = ((lane & jj) == 0) == ((lane & k) == 0);
                skey = keep_min ? (o < skey ? o : skey) : (o > skey ? o : skey);
            }
    }
    const int my_src = (int)(skey & 63);  // slot lw + lane holds query q0 + lw + my_src

    // A operand: 4 blocks of 16 slots, K steps of 64 bytes
    v4i av[4][KS64];
#pragma unroll
    for (int qb = 0; qb < 4; qb++) {
        const int q = q0 + lw + __shfl(my_src, qb * 16 + j);
        const bool ok = q < a.nq;
        const int8_t* src = a.qc8 + (int64_t)(ok ? q : 0) * PITCH + 16 * g;
#pragma unroll
        for (int ks = 0; ks < KS64; ks++) av[qb][ks] = ok ? *(const v4i*)(src + ks * 64) : v4i{0, 0, 0, 0};
    }

    // slot i = tid: the wave that owns slot i runs this thread (its query's
    // threshold and bound from the lane that loaded them)
    const uint64_t src_tau = ((uint64_t)(uint32_t)__shfl((int)(my_tau >> 32), my_src) << 32) |
                             (uint32_t)__shfl((int)(uint32_t)my_tau, my_src);
    const float src_bnd = __shfl(my_bnd, my_src);
    if (tid < QG) {
        const int i = tid;
        const int q = q0 + lw + my_src;
        tau_s[i] = src_tau;
        const float b = src_bnd;
        bnd_s[i] = b;
        qmap_s[i] = q;
        cnt_s[i] = 0;
        float pre = SMALL ? loosen_up(b) : loosen_down(b);
        // the loosest of 4 consecutive slots (lanes 4m .. 4m+3)
#pragma unroll
        for (int x = 1; x <= 2; x <<= 1) {
            const float o = __shfl_xor(pre, x);
            pre = SMALL ? fmaxf(pre, o) : fminf(pre, o);
        }
        if ((lane & 3) == 0) pmin_s[i >> 2] = pre;
    }

    __syncthreads();  // query state above is complete
    // retire the A-fragment loads (and the first chunks) here, not at the
    // fragments' first use in the loop
    __builtin_amdgcn_s_waitcnt(0);

    // Pre-filter of query block qb of a row pair: per 16-row block, the
    // lane's best accumulator over its 4 queries, scaled (row scales are >= 0,
    // so that is the best score of the row's 4 pairs), less the loosest bound
    // of those queries (read where it is used, one LDS read); pm[qb] >= 0
    // unless every exact test of the block's pairs in this lane must fail
    // (fma rounds monotonically in each operand).  The slot order keeps the
    // 4 bounds close, so this is nearly as tight as a test per query.  The
    // bounds come from registers (pb, read once per chunk): an LDS read here
    // would make the wait for it also wait for the B fragments read ahead.
    auto load_pb = [&](float (&pbr)[4]) {
#pragma unroll
        for (int qb = 0; qb < 4; qb++) pbr[qb] = pmin_s[((lw + qb * 16) >> 2) + g];
    };
    float pbr[4];
    auto prefilter = [&](const v4i (&acc)[2][4], const float (&sc)[2], float (&pm)[4], int qb) {
        const float pb = pbr[qb];
        float v[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const v4i x = acc[h][qb];
            const int e = SMALL ? min(min(x[0], x[1]), min(x[2], x[3])) : max(max(x[0], x[1]), max(x[2], x[3]));
            v[h] = SMALL ? __fmaf_rn(-sc[h], (float)e, pb) : __fmaf_rn(sc[h], (float)e, -pb);
        }
        pm[qb] = fmaxf(v[0], v[1]);
    };

    // The pairs of one query block of a row pair that pass the exact test,
    // appended as (pre-score, row) pairs (a wave where one passed the
    // filter): the lane's 8 tests go to a bit mask first, and the appends
    // loop over its set bits, so a lane pays one LDS atomic per pair it
    // appends.  q8 dot pairs are tested against the loosest bound of the
    // lane's 4 queries, already in registers (the slot order keeps it close
    // to each query's own; a pair between the two is a key below the
    // threshold, which the select drops): a triggered block then waits on one
    // LDS round trip, the append's, not two.  Shadow pairs, which the select
    // rescores at a row load each, take each query's own bound (OWNB).
    // Slots without a query have bound +inf (-inf for smallest-k) and sort
    // last; a group of 4 slots whose bounds are all infinite has a NaN
    // loosest bound, which no test passes, and when the query count is not a
    // multiple of 4 (one group then mixes queries and empty slots) the
    // runtime launches the OWNB kernel too, so an empty slot never appends.
    auto survivors = [&](const v4i (&acc)[2][4], int qb, int64_t rb0, const float (&sc)[2]) {
        float bx[4];
        if constexpr (OWNB) {
            const float4 b4 = *(const float4*)&bnd_s[lw + qb * 16 + 4 * g];
            bx[0] = b4.x, bx[1] = b4.y, bx[2] = b4.z, bx[3] = b4.w;
        } else {
            bx[0] = bx[1] = bx[2] = bx[3] = pbr[qb];
        }
        float pv[8];
        uint32_t mask = 0;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const bool valid = rb0 + h * 16 + j < r1;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = fmul_rn(sc[h], (float)acc[h][qb][r]);
                pv[h * 4 + r] = p;
                if (valid && (SMALL ? p <= bx[r] : p >= bx[r])) mask |= 1u << (h * 4 + r);
            }
        }
        while (mask) {
            const int b = __builtin_ctz(mask);
            mask &= mask - 1;
            float p = pv[0];
#pragma unroll
            for (int i = 1; i < 8; i++) p = b == i ? pv[i] : p;
            const int lq = lw + qb * 16 + 4 * g + (b & 3);
            const int pos = atomicAdd(&cnt_s[lq], 1);
            wreg[(uint32_t)(qmap_s[lq] * a.rc + pos)] = dot_pair(p, (uint32_t)(rb0 + (b >> 2) * 16 + j));
        }
    };
    // Exact tests of the query blocks of a row pair whose pre-filter passed
    // in some lane (rare once the bounds are tight).
    auto check = [&](const v4i (&acc)[2][4], int64_t rb0, const float (&sc)[2], const float (&pm)[4]) {
        if (__ballot(fmaxf(fmaxf(pm[0], pm[1]), fmaxf(pm[2], pm[3])) >= 0.0f)) {
#pragma unroll
            for (int qb = 0; qb < 4; qb++)
                if (__ballot(pm[qb] >= 0.0f)) survivors(acc, qb, rb0, sc);
        }
    };
    // B fragments of K step ks of the row pair at tile row row0
    auto load_b = [&](v4i (&b)[2], const uint8_t* tile, int row0, int ks) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int row = row0 + h * 16 + j;
            b[h] = *(const v4i*)(tile + row * PITCH + (((ks * 4 + g) ^ ((row >> 1) & 7)) * 16));
        }
    };
    // MFMAs of the row pair at tile row row0 into acc (its first fragments
    // already in bc), with the pre-filter of the other pair (oacc, osc)
    // spread over the K steps: its VALU work issues while the matrix cores
    // run.  B fragments are read one K step ahead, the last step reading the
    // first fragments of the pair at next0 (if any) into bc (the scheduling
    // barrier keeps the compiler from hoisting every step's reads, which
    // would hold all 2*KS64 fragments in registers).
    auto mfma_pair = [&](v4i (&acc)[2][4], v4i (&bc)[2], const uint8_t* tile, int row0, int next0,
                         const v4i (&oacc)[2][4], const float (&osc)[2], float (&pm)[4]) {
        v4i bn[2];
#pragma unroll
        for (int ks = 0; ks < KS64; ks++) {
            if (ks + 1 < KS64) load_b(bn, tile, row0, ks + 1);
            else if (next0 >= 0) load_b(bn, tile, next0, 0);
#pragma unroll
            for (int qb = 0; qb < 4; qb++)
#pragma unroll
                for (int h = 0; h < 2; h++)
                    acc[h][qb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[qb][ks], bc[h],
                                                                       ks == 0 ? v4i{0, 0, 0, 0} : acc[h][qb], 0, 0, 0);
            if (KS64 >= 4) {
                if (ks < 4) prefilter(oacc, osc, pm, ks);
            } else {
                prefilter(oacc, osc, pm, 2 * ks);
                prefilter(oacc, osc, pm, 2 * ks + 1);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (ks + 1 < KS64 || next0 >= 0) {
                bc[0] = bn[0];
                bc[1] = bn[1];
            }
        }
    };

    if (a.keep_all) {
        // First pass: no threshold exists, so every pair is kept.  Each
        // lane stores its pairs straight to the slot the row's offset in the
        // range gives (16 lanes of a query and row block write 128
        // contiguous bytes); the region counts are the range's rows.
        int buf = 0;
        for (int64_t c0 = r0; c0 < r1; c0 += CH, buf = buf == NBUF - 1 ? 0 : buf + 1) {
            if (sw >= 0)
                mq_wait_barrier<LPW + 1, NBUF - 2>((r1 - c0 - 1) / CH);
            else
                mq_wait_barrier<LPW, NBUF - 2>((r1 - c0 - 1) / CH);
            if (c0 + (NBUF - 1) * CH < r1) issue_chunk(c0 + (NBUF - 1) * CH, buf == 0 ? NBUF - 1 : buf - 1);
            const uint8_t* tile = tiles + buf * TILE;
            const float* cs = cscale + buf * CH;
#pragma unroll
            for (int p = 0; p < PPW; p++) {
                const int row0 = rw + 32 * p;
                v4i acc[2][4];
#pragma unroll
                for (int ks = 0; ks < KS64; ks++) {
                    v4i b[2];
                    load_b(b, tile, row0, ks);
#pragma unroll
                    for (int qb = 0; qb < 4; qb++)
#pragma unroll
                        for (int h = 0; h < 2; h++)
                            acc[h][qb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[qb][ks], b[h],
                                                                               ks == 0 ? v4i{0, 0, 0, 0} : acc[h][qb],
                                                                               0, 0, 0);
                }
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int64_t row = c0 + row0 + h * 16 + j;
                    const float sc = cs[row0 + h * 16 + j];
                    if (row < r1) {
#pragma unroll
                        for (int qb = 0; qb < 4; qb++)
#pragma unroll
                            for (int r = 0; r < 4; r++) {
                                const int q = qmap_s[lw + qb * 16 + 4 * g + r];
                                if (q < a.nq)
                                    wreg[(uint32_t)(q * a.rc) + (uint32_t)(row - r0)] =
                                        dot_pair(fmul_rn(sc, (float)acc[h][qb][r]), (uint32_t)row);
                            }
                    }
                }
            }
        }
        for (int i = tid; i < QG; i += kMq8Threads)
            if (qmap_s[i] < a.nq) a.counts[(int64_t)blockIdx.x * a.nq + qmap_s[i]] = (int)(r1 - r0);
        return;
    }

    // A wave's row pairs of a chunk alternate between the accumulator sets
    // accs[0] and accs[1]; each pair's filter runs under the next pair's
    // MFMAs, the chunk's last pair under the next chunk's first.  Before the
    // first chunk accs[1] holds no pair: its NaN scales make every pre-filter
    // value NaN, which no ballot passes (the filter stays unconditional, so
    // the compiler keeps it among the MFMAs).
    v4i accs[2][2][4];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int qb = 0; qb < 4; qb++) accs[1][h][qb] = v4i{0, 0, 0, 0};
    float scs[2][2] = {{0.0f, 0.0f}, {__builtin_nanf(""), __builtin_nanf("")}};
    int64_t rbs[2] = {r1, r1};  // first row of each set's pair
    float pm[4];

    int buf = 0, par = 0;
    for (int64_t c0 = r0; c0 < r1; c0 += CH, buf = buf == NBUF - 1 ? 0 : buf + 1, par ^= 1) {
        // Flag regions that might not take 2.5 more chunks of keys.  Between
        // two compactions (after the barriers of chunks c and c+1) each wave
        // appends the pairs of PPW row pairs, the previous chunk's last and
        // this chunk's others: one chunk of rows over the WS waves that share
        // a query.  A count read here may miss up to one such window, the
        // window up to the next compaction adds one chunk, and after the
        // last chunk the pending last pairs add at most half a chunk.  The
        // runtime sizes regions rc >= k + 2.5*CH, so a compacted region (k
        // pairs) is never flagged again at once.
        if (wave_s < NFW) {
            // (slot index from the scalar wave index and the lane count, so
            // the compiler recomputes it instead of spilling it)
            const int ln = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0));
            const uint64_t m = __ballot(cnt_s[wave_s * 64 + ln] > a.rc - (5 * CH) / 2);
            if (ln == 0) flags[par][wave_s] = m;
        }
        // this wave's loads of chunk c are done once at most the loads of
        // the chunks issued after it are outstanding; the barrier extends
        // that to every wave, retires the previous chunk's reads of the tile
        // about to be refilled, and publishes the flags
        // (the scale-loading waves issue one more load per chunk)
        if (sw >= 0)
            mq_wait_barrier<LPW + 1, NBUF - 2>((r1 - c0 - 1) / CH);
        else
            mq_wait_barrier<LPW, NBUF - 2>((r1 - c0 - 1) / CH);
        const int nbuf = buf == 0 ? NBUF - 1 : buf - 1;  // tile of chunk c+NBUF-1 (free now)
        const uint8_t* tile = tiles + buf * TILE;
        const float* cs = cscale + buf * CH;
        // the first pair's first fragments and the bounds go out with the
        // flags' read (a compaction writes neither this tile nor the
        // fragments; it reloads the bounds it may change)
        v4i bc[2];
        load_b(bc, tile, rw, 0);
        load_pb(pbr);
        {
            bool any = false;
#pragma unroll
            for (int w = 0; w < NFW; w++) any |= flags[par][w] != 0;
            if (any) {
                // rare: compact full regions to their best k pairs (the
                // scratch tile holds the region's keys, then its pairs).
                // Every wave's appends (global stores, which the barrier's
                // vmcnt wait above may leave in flight) are complete before
                // any wave reads a region: the workgroup shares one L1, so
                // vmcnt(0) and a barrier order them.
                __builtin_amdgcn_s_waitcnt(0);
                __syncthreads();
                uint64_t* skeys = (uint64_t*)(tiles + nbuf * TILE);
                uint64_t* spairs = skeys + a.rc;
                for (int lq = 0; lq < QG; lq++) {
                    if (!((flags[par][lq >> 6] >> (lq & 63)) & 1)) continue;
                    const int qx = qmap_s[lq];
                    uint64_t* reg = wreg + (uint32_t)(qx * a.rc);
                    const int c = cnt_s[lq];
                    for (int i = tid; i < c; i += kMq8Threads) {
                        const uint64_t e = reg[i];
                        spairs[i] = e;
                        if (SHADOW) {
                            // the exact q4 score of the pair's row
                            const int64_t q = qx;
                            const float sc = q4_exact_score(a.op, a.q4codes, a.q4scales, a.dnorm, a.dd, a.d,
                                                            (int64_t)(uint32_t)e, (const int*)(a.qhi + q * a.d),
                                                            (const int*)(a.qlo + q * a.d), a.qconst[q]);
                            skeys[i] = make_key(sc, (uint32_t)e, SMALL);
                        } else {
                            skeys[i] = dot_pair_key(e, a.qconst[qx].a, SMALL);
                        }
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
                            bnd_s[lq] = SHADOW ? shadow_bound(minkey, a.qbound[2 * qx], a.qbound[2 * qx + 1], SMALL)
                                               : mq_bound<OP_DOT>(minkey, a.qconst[qx], SMALL);
                            const int m0 = lq & ~3;
                            float pre = SMALL ? loosen_up(bnd_s[m0]) : loosen_down(bnd_s[m0]);
                            for (int x = 1; x < 4; x++) {
                                const float o = SMALL ? loosen_up(bnd_s[m0 + x]) : loosen_down(bnd_s[m0 + x]);
                                pre = SMALL ? fmaxf(pre, o) : fminf(pre, o);
                            }
                            pmin_s[lq >> 2] = pre;
                        }
                    }
                    __syncthreads();
                }
                load_pb(pbr);
            }
        }
        // pair p into accs[p & 1], under which pair p-1 (the previous
        // chunk's last for p = 0) is filtered
#pragma unroll
        for (int p = 0; p < PPW; p++) {
            const int cur = p & 1, oth = cur ^ 1;
            const int row0 = rw + 32 * p;
            // this pair's scales, read before its MFMAs: the next pair's
            // filter uses them, long after they arrive
            scs[cur][0] = cs[row0 + j];
            scs[cur][1] = cs[row0 + 16 + j];
            mfma_pair(accs[cur], bc, tile, row0, p + 1 < PPW ? row0 + 32 : -1, accs[oth], scs[oth], pm);
            // Chunk c+NBUF-1's loads (into the tile chunk c-1 left, which the
            // barrier released and any compaction above has finished with)
            // go out once the first pair's MFMAs are queued: issued right
            // after the barrier, every wave's burst held the MFMAs back (C4:
            // 3-42 us less scan per step on three boxes, never more).
            if (p == 0 && c0 + (NBUF - 1) * CH < r1) issue_chunk(c0 + (NBUF - 1) * CH, nbuf);
            check(accs[oth], rbs[oth], scs[oth], pm);
            rbs[cur] = c0 + row0;
        }
    }
    // the last chunk's last pair
    load_pb(pbr);
#pragma unroll
    for (int qb = 0; qb < 4; qb++) prefilter(accs[1], scs[1], pm, qb);
    check(accs[1], rbs[1], scs[1], pm);
    __syncthreads();
    for (int i = tid; i < QG; i += kMq8Threads)
        if (qmap_s[i] < a.nq) a.counts[(int64_t)blockIdx.x * a.nq + qmap_s[i]] = cnt_s[i];
}

// ------------------------------------------------------ q4 int8 shadow
//
// A q4 row x (x_j = f16 scale of j's block times its nibble code) gets int8
// codes e_j = round(x_j / t) with t = maxabs(x) / 127 and the per-row scales
// t (dot) and t / dnorm (cosine).  The shadow scan ranks rows by
// p = scale * (e . c) against full-range int8 query codes c and keeps every
// row the exact q4 score could place in the top k: with E = |x - t e| and
// F = t |e|, |x . q - t e . qa c| <= E |q| + F |q - qa c|, so per-row error
// bounds need only E, F (and |x| for cosine) -- their maxima over the rows
// go to ShadowInfo.

// An f32 at least v >= 0 (the cast rounds to nearest; the factor covers it).
__device__ __forceinline__ float f32_up(double v) { return (float)(v * (1.0 + 9.5367431640625e-7)); }

__global__ void shadow_info_clear_kernel(ShadowInfo* info) {
    if (threadIdx.x < 8) (&info->me_cos)[threadIdx.x] = 0u;
}

// One wave per row (grid-stride); lane i holds bytes i, i+64, i+128 of the
// packed row, i.e. elements 2i and 2i+1 of each (d <= 384).
__global__ __launch_bounds__(256) void q4_shadow_build_kernel(const uint8_t* __restrict__ packed,
                                                              const uint16_t* __restrict__ scales,
                                                              const float* __restrict__ dnorm, int64_t n, int d,
                                                              int spitch, int8_t* __restrict__ codes,
                                                              float* __restrict__ sc_dot, float* __restrict__ sc_cos,
                                                              ShadowInfo* __restrict__ info) {
    const int lane = threadIdx.x & 63;
    const int64_t nw = (int64_t)gridDim.x * 4;
    const int hb = d / 2;
    const int nb = d / 32;
    float me_c = 0.0f, mf_c = 0.0f, me_d = 0.0f, mf_d = 0.0f, mn = 0.0f;
    for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < n; row += nw) {
        float x[3][2];
        float m = 0.0f;
#pragma unroll
        for (int u = 0; u < 3; u++) {
            const int i = lane + 64 * u;
            x[u][0] = x[u][1] = 0.0f;
            if (i < hb) {
                const int byte = packed[row * hb + i];
                const float sc = h2f(scales[row * nb + (2 * i) / 32]);
                // f16 significand (11 bits) times a 4-bit code: exact in f32
                x[u][0] = fmul_rn(sc, (float)((int)(int8_t)(byte << 4) >> 4));
                x[u][1] = fmul_rn(sc, (float)((int)(int8_t)byte >> 4));
                m = fmaxf(m, fmaxf(__builtin_fabsf(x[u][0]), __builtin_fabsf(x[u][1])));
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        const float t = fdiv_rn(m, 127.0f);
        double e2 = 0.0, f2 = 0.0, n2 = 0.0;
        int8_t* crow = codes + row * spitch;
#pragma unroll
        for (int u = 0; u < 3; u++) {
            const int i = lane + 64 * u;
            if (i >= hb) continue;
            int e[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const double xv = (double)x[u][h];
                int c = 0;
                if (t > 0.0f) {
                    const double r = __builtin_rint(xv / (double)t);
                    c = (int)(r > 127.0 ? 127.0 : (r < -127.0 ? -127.0 : r));
                }
                e[h] = c;
                const double ex = xv - (double)t * (double)c;
                e2 += ex * ex;
                f2 += (double)(c * c);
                n2 += xv * xv;
            }
            *(uint16_t*)(crow + 2 * i) = (uint16_t)((uint8_t)e[0] | ((uint16_t)(uint8_t)e[1] << 8));
        }
        for (int c = d + 2 * lane; c < spitch; c += 128) *(uint16_t*)(crow + c) = 0;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            e2 += __shfl_xor(e2, off);
            f2 += __shfl_xor(f2, off);
            n2 += __shfl_xor(n2, off);
        }
        if (lane == 0) {
            const float dn = dnorm[row];
            sc_dot[row] = t;
            sc_cos[row] = dn > 0.0f ? fdiv_rn(t, dn) : 0.0f;
        }
        const double E = __builtin_sqrt(e2), F = (double)t * __builtin_sqrt(f2), N = __builtin_sqrt(n2);
        me_d = fmaxf(me_d, f32_up(E));
        mf_d = fmaxf(mf_d, f32_up(F));
        mn = fmaxf(mn, f32_up(N));
        if (N > 0.0) {
            me_c = fmaxf(me_c, f32_up(E / N));
            mf_c = fmaxf(mf_c, f32_up(F / N));
        }
    }
    // workgroup maxima, then one atomic per value that raises the global one
    __shared__ float red[4][5];
    if (lane == 0) {
        const int w = threadIdx.x >> 6;
        red[w][0] = me_c, red[w][1] = mf_c, red[w][2] = me_d, red[w][3] = mf_d, red[w][4] = mn;
    }
    __syncthreads();
    if (threadIdx.x < 5) {
        const int i = threadIdx.x;
        const float v = fmaxf(fmaxf(red[0][i], red[1][i]), fmaxf(red[2][i], red[3][i]));
        unsigned int* dst = &info->me_cos + i;
        if (__float_as_uint(v) > *(volatile unsigned int*)dst) atomicMax(dst, __float_as_uint(v));
    }
}

hipError_t launch_shadow_info_clear(ShadowInfo* info, hipStream_t s) {
    hipLaunchKernelGGL(shadow_info_clear_kernel, dim3(1), dim3(64), 0, s, info);
    return hipGetLastError();
}

hipError_t launch_q4_shadow_build(const uint8_t* packed, const uint16_t* scales, const float* dnorm, int64_t n,
                                  int d, int spitch, int8_t* codes, float* sc_dot, float* sc_cos,
                                  ShadowInfo* info, hipStream_t s) {
    if (d % 32 != 0 || d > 384 || spitch < d || spitch % 2 != 0) return hipErrorInvalidValue;
    const int64_t wgs = std::min<int64_t>(8192, (n + 3) / 4);
    hipLaunchKernelGGL(q4_shadow_build_kernel, dim3((unsigned)wgs), dim3(256), 0, s, packed, scales, dnorm, n, d,
                       spitch, codes, sc_dot, sc_cos, info);
    return hipGetLastError();
}

// pitch 512 would exceed the register budget (A fragments alone take 128)
bool mq8_supported(int pitch) { return pitch == 128 || pitch == 256 || pitch == 384; }

MqShape mq8_shape(int pitch, int ws, bool shadow) {
    MqShape s;
    s.kind = 1;
    s.ks = pitch / 64;
    s.na = 4;
    s.wq = kMq8Waves / ws;
    s.ws = ws;
    s.shadow = shadow ? 1 : 0;
    s.qg = kMq8QG / ws;
    s.chunk = kMq8CH * ws;  // the kernel's CH
    s.tile = s.chunk * pitch;
    s.tile_bytes = mq8_nbuf(s.tile, s.qg, s.chunk) * (s.tile + s.chunk * 4);  // chunk tiles + row scales
    s.threads = kMq8Threads;
    return s;
}

template <int KS64, bool SMALL, int WS, bool SHADOW, bool OWNB>
static hipError_t launch_mq8_one(const MqArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)mq8_scan_kernel<KS64, SMALL, WS, SHADOW, OWNB>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL((mq8_scan_kernel<KS64, SMALL, WS, SHADOW, OWNB>), grid, dim3(kMq8Threads), lds, s, a);
    return hipGetLastError();
}

template <int KS64>
static hipError_t launch_mq8_ks(const MqShape& sh, const MqArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    const bool sm = a.smallest != 0;
    // each query's own bound in the exact test: shadow pairs, and query
    // counts that leave a group of 4 slots partly empty
    const bool own = sh.shadow != 0 || (a.nq & 3) != 0;
#define MANTA_MQ8(SM, W, SH, OB)                                                  \
    if (sm == SM && sh.ws == W && (sh.shadow != 0) == SH && own == OB)            \
        return launch_mq8_one<KS64, SM, W, SH, OB>(a, grid, lds, s);
    MANTA_MQ8(false, 1, false, false)
    MANTA_MQ8(true, 1, false, false)
    MANTA_MQ8(false, 2, false, false)
    MANTA_MQ8(true, 2, false, false)
    MANTA_MQ8(false, 1, true, true)
    MANTA_MQ8(true, 1, true, true)
    MANTA_MQ8(false, 2, true, true)
    MANTA_MQ8(true, 2, true, true)
    MANTA_MQ8(false, 1, false, true)
    MANTA_MQ8(true, 1, false, true)
    MANTA_MQ8(false, 2, false, true)
    MANTA_MQ8(true, 2, false, true)
#undef MANTA_MQ8
    return hipErrorInvalidValue;
}

hipError_t launch_mq8_scan(const MqShape& sh, const MqArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    switch (sh.ks) {
        case 2: return launch_mq8_ks<2>(sh, a, grid, lds, s);
        case 4: return launch_mq8_ks<4>(sh, a, grid, lds, s);
        case 6: return launch_mq8_ks<6>(sh, a, grid, lds, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace manta
