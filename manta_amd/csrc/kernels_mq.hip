// kernels_mq.hip -- many queries against one shared q8 candidate matrix
// ([Q,D] x [N,D]) on the i8 matrix cores of gfx950.
//
// mq_scan_kernel: workgroup = 4 waves, grid = (row ranges, query groups).
// Each wave keeps NA blocks of query codes resident in VGPRs as the A
// operand of v_mfma_i32_32x32x32_i8 (32 A rows = 32 queries for E8 codes,
// or 16 queries x {hi, lo} digit for E16 codes).  Candidate rows stream
// through LDS in chunks of 32 rows per wave: a chunk is one contiguous span
// of HBM, moved by direct-to-LDS loads into a padded tile two to four chunks
// ahead of its use, and every wave reads its B fragments from there -- with
// the waves splitting the queries (WQ = 4) each candidate byte is fetched
// once per workgroup and feeds 4*NA MFMAs.
//
// With the candidate on the MFMA output column, lane l ends a 32-row block
// holding candidate l%32 against 16 A rows: 16 queries (E8), or 8 queries as
// (hi, lo) pairs in acc[r] / acc[r+4] (E16; A rows [hi q0-7 | lo q0-7 |
// hi q8-15 | lo q8-15]), combined exactly as fma(256, hi, lo).
//
// Top-k runs in passes over growing row prefixes.  A pass gets a threshold
// key per query -- the k-th best key of all rows of the earlier passes, a
// valid lower bound of the final k-th key -- and appends every key above it
// to a per-(query, workgroup) region in HBM.  A cheap monotone pre-score
// (dot: s*acc, l2: dist^2, cosine: q.d against tau*|q|*|d|) tested against
// a loosened bound decides which scores are computed exactly.  If a region
// still fills up (adversarially ordered rows) the workgroup compacts it to
// its best k keys and raises its own threshold, so no key is ever lost.
// mq_select_kernel then merges the previous best k with the pass's regions
// into the new best k and the next pass's threshold.
#include "mq_common.hpp"
#include "q4_common.hpp"

namespace manta {

template <int OP, int ENC, int KS, int NA, int WQ, int MODE, bool SMALL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void mq_scan_kernel(MqArgs a) {
    constexpr int PITCH = KS * 32;           // bytes per candidate row
    constexpr int P = PITCH + 16;            // LDS row pitch (padding spreads banks)
    constexpr int WR = 4 / WQ;               // waves splitting the rows of a chunk (WQ: 1, 2 or 4)
    // One 32-row block per wave per chunk (WR*32 rows), two workgroups per
    // CU: chunks c+1 .. c+NBUF-1 are in flight while chunk c is multiplied.
    constexpr int CHUNK = WR * 32;                   // rows per chunk
    constexpr int SEGS = (CHUNK * P + 1023) / 1024;  // 1 KB LDS segments per chunk tile
    constexpr int DPW = (SEGS + 3) / 4;              // 16-byte direct-to-LDS loads per wave per chunk
    constexpr int TILE = DPW * 4 * 1024;             // LDS bytes per tile
    constexpr int NARR = (OP == OP_DOT || OP == OP_DOT16) ? 1 : 2;  // per-row arrays: scale (+ |d| or |d|^2)
    constexpr int CSA = (CHUNK + 63) / 64;           // 256-byte segments per array per chunk
    constexpr int CPW = (NARR * CSA + 3) / 4;        // 4-byte direct-to-LDS loads per wave per chunk
    constexpr int CTILE = CPW * 4 * 256;             // LDS bytes of a chunk's per-row constants
    constexpr int VPW = DPW + CPW;                   // direct-to-LDS loads per wave per chunk
    constexpr int NBUF = mq_nbuf(TILE + CTILE, VPW); // LDS chunk tiles
    constexpr int QPB = ENC == MQ_E8 ? 32 : 16;  // queries per A block
    constexpr int QPW = NA * QPB;                // queries per wave
    constexpr int QG = WQ * QPW;                 // queries per workgroup
    constexpr int QPL = ENC == MQ_E8 ? 16 : 8;   // queries per lane per A block
    constexpr int NC = (NA == 1 && KS >= 4) ? 2 : 1;  // accumulator chains per A block
    constexpr int NFW = (QG + 63) / 64;               // flag words
    constexpr bool APPEND = MODE == MQ_APPEND;

    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* tiles = smem;                                   // [NBUF][TILE]
    float* consts = (float*)(smem + NBUF * TILE);            // [NBUF][CTILE / 4]
    // compaction scratch: the tile that is about to be refilled, or an extra
    // LDS area when rc keys do not fit in a tile
    uint64_t* scratch_extra = (uint64_t*)(smem + NBUF * (TILE + CTILE));
    __shared__ uint64_t tau_s[QG];
    // per-query values the epilogue reads four at a time (float4)
    __shared__ __attribute__((aligned(16))) float bnd_s[QG];  // pre-score bound
    __shared__ __attribute__((aligned(16))) float qa_s[QG];   // QConst.a
    __shared__ __attribute__((aligned(16))) float qc_s[QG];   // QConst.c
    __shared__ int cnt_s[QG];
    __shared__ uint64_t flags[2][NFW];  // double-buffered by chunk parity
    __shared__ RadixShared ss;
    __shared__ int wpos;
    __shared__ unsigned long long minkey;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int half = lane >> 5;
    const int wq = wave % WQ;
    const int wr = wave / WQ;
    const int q0 = blockIdx.y * QG;

    // ---- query constants, thresholds, region counters
    for (int i = tid; i < QG; i += 256) {
        const int q = q0 + i;
        const bool ok = q < a.nq;
        const QConst qc = ok ? a.qconst[q] : QConst{1.0f, 0.0f, 0.0f, 0.0f};
        qa_s[i] = qc.a;
        qc_s[i] = qc.c;
        const uint64_t tk = (APPEND && ok) ? a.tau[q] : 0ull;
        // a query past nq gets a bound nothing passes and the largest key
        tau_s[i] = ok ? tk : ~0ull;
        bnd_s[i] = ok ? mq_bound<OP>(tk, qc, SMALL) : (SMALL ? -__builtin_inff() : __builtin_inff());
        cnt_s[i] = 0;
    }

    // ---- A operand: this wave's query codes, resident for the whole scan
    v4i av[NA][KS];
#pragma unroll
    for (int na = 0; na < NA; na++) {
        const int i = lane & 31;
        int q;
        const int8_t* plane;
        if (ENC == MQ_E8) {
            q = q0 + wq * QPW + na * 32 + i;
            plane = a.qc8;
        } else {
            const int blk = i >> 3;  // 0: hi q0-7, 1: lo q0-7, 2: hi q8-15, 3: lo q8-15
            q = q0 + wq * QPW + na * 16 + (blk >> 1) * 8 + (i & 7);
            plane = (blk & 1) ? a.qlo : a.qhi;
        }
        const bool ok = q < a.nq;
        const int8_t* src = plane + (int64_t)(ok ? q : 0) * PITCH + half * 16;
#pragma unroll
        for (int s = 0; s < KS; s++) av[na][s] = ok ? *(const v4i*)(src + s * 32) : v4i{0, 0, 0, 0};
    }

    // slot u of A block na -> accumulator index and workgroup-local query
    auto slot_r = [](int u) { return ENC == MQ_E8 ? u : (u < 4 ? u : u + 4); };
    auto slot_lq = [&](int na, int u) {
        const int r = slot_r(u);
        const int i = 8 * (r / 4) + 4 * half + (r % 4);
        return wq * QPW + na * QPB + (ENC == MQ_E8 ? i : (i >> 4) * 8 + (i & 7));
    };
    uint32_t live[NA];  // slots whose query exists
#pragma unroll
    for (int na = 0; na < NA; na++) {
        live[na] = 0;
#pragma unroll
        for (int u = 0; u < QPL; u++)
            if (q0 + slot_lq(na, u) < a.nq) live[na] |= 1u << u;
    }

    // this workgroup's key regions: [query][rc] (32-bit indices, checked on the host)
    uint64_t* wreg = a.regions + (int64_t)blockIdx.x * a.nq * a.rc;
    const int64_t r0 = a.row_begin + (int64_t)blockIdx.x * a.rows_per_wg;
    int64_t r1 = r0 + a.rows_per_wg;
    if (r1 > a.row_end) r1 = a.row_end;

    // Candidate chunks go straight from HBM into LDS tiles (16-byte direct-
    // to-LDS loads, no VGPR staging) NBUF-1 chunks ahead of their use.  Lane
    // i of a wave's load fills bytes [16i, 16i+16) of a 1 KB tile segment;
    // the source is the row byte that belongs there in the padded layout,
    // clamped into the range (padding and rows past the range receive
    // arbitrary in-range bytes and are never used).  The chunk's per-row
    // constants follow the same way (4-byte loads, 64 rows per load), so the
    // loop issues no other global loads that would have to be waited for.
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);
    auto issue_chunk = [&](int64_t c0, int buf) {
        const int8_t* base = a.codes + c0 * PITCH;
        const int left = (int)(r1 - c0 < CHUNK ? r1 - c0 : CHUNK);
        const int lim = left * PITCH - 16;  // last 16 bytes inside the range
        const uint32_t t = lds_addr(tiles) + buf * TILE;
#pragma unroll
        for (int i = 0; i < DPW; i++) {
            const int seg = wave_s * DPW + i;
            const int x = seg * 1024 + lane * 16;
            const int row = x / P;
            const int off = row * PITCH + (x - row * P);
            lds_load16(base + (off < lim ? off : lim), t + seg * 1024);
        }
        const uint32_t ct = lds_addr(consts) + buf * CTILE;
#pragma unroll
        for (int i = 0; i < CPW; i++) {
            const int cs = wave_s * CPW + i;  // segments past NARR*CSA are filler
            const int arr = cs / CSA < NARR ? cs / CSA : 0;
            const int row = (cs % CSA) * 64 + lane;
            const float* src = arr == 0 ? a.scales : (OP == OP_COSINE ? a.dnorm : a.dd);
            lds_load4(src + c0 + (row < left ? row : left - 1), ct + cs * 256);
        }
    };
    __syncthreads();  // LDS query state above is complete
    // Retire the A-fragment loads here, where the compiler sees it: otherwise
    // it would wait for them (and with them every chunk load in flight) at
    // their first use inside the loop, in every iteration.
    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int j = 0; j < NBUF - 1; j++)
        if (r0 + j * CHUNK < r1) issue_chunk(r0 + j * CHUNK, j);

    // MFMAs of one 32-row block: B fragments from the LDS tile, A resident.
    auto multiply = [&](const uint8_t* tile, v16i (&acc)[NA]) {
        v16i ch[NA][NC];
#pragma unroll
        for (int na = 0; na < NA; na++)
#pragma unroll
            for (int c = 0; c < NC; c++)
#pragma unroll
                for (int r = 0; r < 16; r++) ch[na][c][r] = 0;
        const uint8_t* bp = tile + (wr * 32 + (lane & 31)) * P + half * 16;
#pragma unroll
        for (int s = 0; s < KS; s++) {
            const v4i bf = *(const v4i*)(bp + s * 32);
#pragma unroll
            for (int na = 0; na < NA; na++)
                ch[na][s % NC] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[na][s], bf, ch[na][s % NC], 0, 0, 0);
        }
#pragma unroll
        for (int na = 0; na < NA; na++) {
            acc[na] = ch[na][0];
            if (NC > 1) acc[na] += ch[na][NC - 1];
        }
    };

    // Per-query values of one A block's slots: slot u's query is
    // lq = lq0 + 8*(u/4) + u%4, so four slots read one float4 from LDS.
    struct SlotVals {
        float bq[QPL], qa[QPL], qcv[QPL];
    };
    auto slot_vals = [&](int na, SlotVals& v) {
        const int lq0 = wq * QPW + na * QPB + 4 * half;
#pragma unroll
        for (int m = 0; m < QPL / 4; m++) {
            const float4 b4 = *(const float4*)&bnd_s[lq0 + 8 * m];
            v.bq[4 * m] = b4.x, v.bq[4 * m + 1] = b4.y, v.bq[4 * m + 2] = b4.z, v.bq[4 * m + 3] = b4.w;
            if (OP != OP_DOT) {
                const float4 a4 = *(const float4*)&qa_s[lq0 + 8 * m];
                v.qa[4 * m] = a4.x, v.qa[4 * m + 1] = a4.y, v.qa[4 * m + 2] = a4.z, v.qa[4 * m + 3] = a4.w;
            }
            if (OP == OP_L2) {
                const float4 c4 = *(const float4*)&qc_s[lq0 + 8 * m];
                v.qcv[4 * m] = c4.x, v.qcv[4 * m + 1] = c4.y, v.qcv[4 * m + 2] = c4.z, v.qcv[4 * m + 3] = c4.w;
            }
        }
    };
    // pre-scores: dot s*acc, l2 dist^2, cosine q.d (exact f32 steps)
    auto pre_of = [&](const v16i& accs, const SlotVals& v, int u, float scale, float rowc) {
        const int r = slot_r(u);
        if (OP == OP_DOT) return fmul_rn(scale, (float)accs[r]);
        const float dotf = __fmaf_rn(256.0f, (float)accs[r], (float)accs[r + 4]);
        const float qd = fmul_rn(fmul_rn(scale, v.qa[u]), dotf);
        return OP == OP_L2 ? fsub_rn(fadd_rn(v.qcv[u], rowc), fmul_rn(2.0f, qd)) : qd;
    };
    auto keep_of = [&](const SlotVals& v, int u, float p, float rowc) {
        const float bv = OP == OP_COSINE ? fmul_rn(v.bq[u], rowc) : v.bq[u];
        return SMALL ? !(p > bv) : !(p < bv);
    };
    auto score_of = [&](float p, int lq, float rowc) {
        if (OP == OP_DOT) return fdiv_rn(fmul_rn(p, qa_s[lq]), 127.0f);
        if (OP == OP_DOT16) return p;
        if (OP == OP_COSINE) {
            const float den = fmul_rn(a.qconst[q0 + lq].b, rowc);
            return den == 0.0f ? 0.0f : fdiv_rn(p, den);
        }
        return fsqrt_rn(p < 0.0f ? 0.0f : p);
    };
    // Branch-free filter of one block: does any slot of this lane pass?
    auto filter_any = [&](const v16i (&acc)[NA], int64_t row, float scale, float rowc) {
        bool any = false;
#pragma unroll
        for (int na = 0; na < NA; na++) {
            SlotVals v;
            slot_vals(na, v);
#pragma unroll
            for (int u = 0; u < QPL; u++) any |= keep_of(v, u, pre_of(acc[na], v, u, scale, rowc), rowc);
        }
        return any && row < r1;
    };
    // Exact scores and keys of the survivors (a wave with at least one).
    auto survivors = [&](const v16i (&acc)[NA], int64_t row, float scale, float rowc) {
        if (row >= r1) return;
#pragma unroll
        for (int na = 0; na < NA; na++) {
            SlotVals v;
            slot_vals(na, v);
#pragma unroll
            for (int u = 0; u < QPL; u++) {
                const float p = pre_of(acc[na], v, u, scale, rowc);
                if (keep_of(v, u, p, rowc) && ((live[na] >> u) & 1)) {
                    const int lq = slot_lq(na, u);
                    // (no comparison with the threshold key: the bound test
                    // is at most an ulp looser, and the select merges with k
                    // keys above the threshold, which such a key cannot
                    // displace; live excludes the padding queries)
                    const uint64_t key = make_key(score_of(p, lq, rowc), (uint32_t)row, SMALL);
                    const int pos = atomicAdd(&cnt_s[lq], 1);
                    wreg[(uint32_t)((q0 + lq) * a.rc + pos)] = key;
                }
            }
        }
    };
    // Score-matrix stores of one block.
    auto store_scores = [&](const v16i (&acc)[NA], int64_t row, float scale, float rowc) {
        if (row >= r1) return;
#pragma unroll
        for (int na = 0; na < NA; na++) {
            SlotVals v;
            slot_vals(na, v);
#pragma unroll
            for (int u = 0; u < QPL; u++) {
                if (!((live[na] >> u) & 1)) continue;
                const int lq = slot_lq(na, u);
                a.out_scores[(int64_t)(q0 + lq) * a.n + row] = score_of(pre_of(acc[na], v, u, scale, rowc), lq, rowc);
            }
        }
    };
    int buf = 0, par = 0;
    for (int64_t c0 = r0; c0 < r1; c0 += CHUNK, buf = buf == NBUF - 1 ? 0 : buf + 1, par ^= 1) {
        if (APPEND) {
            // Flag regions that might not take one more chunk of keys.  Read
            // before the barrier, a count may still miss up to CHUNK keys of
            // the chunk other waves are filtering, hence the margin of two
            // chunks (rc >= k + 2*CHUNK + 1).  Parity buffers: the flags
            // written here are read after this barrier, while the next
            // chunk's flags go to the other buffer.
            for (int w = wave; w < NFW; w += 4) {
                const int i = w * 64 + lane;
                const uint64_t m = __ballot(i < QG && cnt_s[i < QG ? i : 0] > a.rc - 2 * CHUNK);
                if (lane == 0) flags[par][w] = m;
            }
        }
        // This wave's loads of chunk c are done once at most the loads of the
        // chunks issued after it are outstanding (loads complete in order);
        // the barrier extends that to every wave's loads, retires the
        // previous chunk's tile reads before that tile is refilled, and
        // publishes the flags.  (A plain __syncthreads would wait for every
        // chunk in flight.)
        mq_wait_barrier<VPW, NBUF - 2>((r1 - c0 - 1) / CHUNK);
        const int nbuf = buf == 0 ? NBUF - 1 : buf - 1;  // tile of chunk c+NBUF-1 (free now)
        if (APPEND) {
            // rare: compact full regions to their best k keys
            bool any = false;
#pragma unroll
            for (int w = 0; w < NFW; w++) any |= flags[par][w] != 0;
            if (any) {
                // every wave's appends (stores the barrier's vmcnt count may
                // leave in flight) are complete before a region is read back:
                // the workgroup shares one L1
                __builtin_amdgcn_s_waitcnt(0);
                __syncthreads();
                uint64_t* scratch = a.rc * 8 <= TILE ? (uint64_t*)(tiles + nbuf * TILE) : scratch_extra;
                for (int lq = 0; lq < QG; lq++) {
                    if (!((flags[par][lq >> 6] >> (lq & 63)) & 1)) continue;
                    uint64_t* reg = wreg + (uint32_t)((q0 + lq) * a.rc);
                    const int c = cnt_s[lq];
                    for (int i = tid; i < c; i += 256) scratch[i] = reg[i];
                    if (tid == 0) {
                        wpos = 0;
                        minkey = ~0ull;
                    }
                    __syncthreads();
                    uint64_t prefix, pmask;
                    block_radix_prefix(scratch, c, a.k, ss, prefix, pmask);
                    uint64_t lo = ~0ull;
                    for (int i = tid; i < c; i += 256) {
                        const uint64_t key = scratch[i];
                        if ((key & pmask) >= prefix) {
                            reg[atomicAdd(&wpos, 1)] = key;
                            lo = key < lo ? key : lo;
                        }
                    }
                    if (lo != ~0ull) atomicMin(&minkey, (unsigned long long)lo);
                    __syncthreads();
                    if (tid == 0) {
                        cnt_s[lq] = a.k;
                        if (minkey > tau_s[lq]) {
                            tau_s[lq] = minkey;
                            bnd_s[lq] = mq_bound<OP>(minkey, a.qconst[q0 + lq], SMALL);
                        }
                    }
                    __syncthreads();
                }
            }
        }

        // Refill the free tile with chunk c+NBUF-1 now -- except that the
        // score matrix does it after this chunk's stores, which also count
        // in vmcnt and would otherwise be waited for with it.
        if (APPEND && c0 + (NBUF - 1) * CHUNK < r1) issue_chunk(c0 + (NBUF - 1) * CHUNK, nbuf);
        const uint8_t* tile = tiles + buf * TILE;
        const float* ctile = consts + buf * (CTILE / 4);
        const int64_t row = c0 + wr * 32 + (lane & 31);
        const float scale = ctile[wr * 32 + (lane & 31)];
        const float rowc = NARR == 1 ? 0.0f : ctile[CSA * 64 + wr * 32 + (lane & 31)];
        // MFMAs of this wave's 32-row block, then its filter: one compare per
        // slot without branches, and the exact scores and keys only in a wave
        // that has a survivor
        v16i acc[NA];
        multiply(tile, acc);
        if (APPEND) {
            if (__ballot(filter_any(acc, row, scale, rowc))) survivors(acc, row, scale, rowc);
        } else {
            store_scores(acc, row, scale, rowc);
        }
        if (!APPEND && c0 + (NBUF - 1) * CHUNK < r1) issue_chunk(c0 + (NBUF - 1) * CHUNK, nbuf);
    }
    if (!APPEND) return;
    __syncthreads();
    for (int i = tid; i < QG; i += 256)
        if (q0 + i < a.nq) a.counts[(int64_t)blockIdx.x * a.nq + q0 + i] = cnt_s[i];
}

// ------------------------------------------------------------- select

// Merge a query's previous best keys with the keys its pass appended: the
// new best k (sorted descending), their count, and the next pass's
// threshold (the k-th key once k keys exist).  One workgroup per query.
// Keys stream through an LDS buffer of NT*16 keys; whenever it fills, a
// radix select keeps the best k.  The final pass writes ids and scores.
template <int NT, int PM>
__global__ __launch_bounds__(NT) void mq_select_kernel(MqSelectArgs a) {
    // PM: region entries are keys (0), q8 dot pairs (1) or shadow pairs (2)
    constexpr int KPT = 16;
    constexpr int LCAP = NT * KPT;
    constexpr int NW = NT / 64;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint64_t* buf = (uint64_t*)smem;           // [LCAP]
    int* pre = (int*)(smem + LCAP * 8);        // [R + 1]
    __shared__ RadixShared rs;
    __shared__ int wsum[NW];
    __shared__ int wpos, wpos2;
    __shared__ int cmax_s;
    __shared__ unsigned long long minkey;
    __shared__ int kpos;
    __shared__ int qh_s[PM == 2 ? kMaxQueryDim / 4 : 1];
    __shared__ int ql_s[PM == 2 ? kMaxQueryDim / 4 : 1];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int q = blockIdx.x;
    const int k = a.k;

    // the previous best's count travels with the region counts (one round trip)
    int fill = __builtin_amdgcn_readfirstlane(a.bcnt[q]);
    // exclusive prefix of the pass's region counts, and their maximum
    int carry = 0, cmax = 0;
    if (tid == 0) cmax_s = 0;
    for (int base = 0; base < a.R; base += NT) {
        const int w = base + tid;
        int c = w < a.R ? a.counts[(int64_t)w * a.nq + q] : 0;
        c = c < a.rc ? c : a.rc;
        cmax = c > cmax ? c : cmax;
        const int incl = wave_incl_scan(c);
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        int before = carry;
        for (int j = 0; j < wave; j++) before += wsum[j];
        if (w < a.R) pre[w] = before + incl - c;
        int total = 0;
        for (int j = 0; j < NW; j++) total += wsum[j];
        carry += total;
        __syncthreads();
    }
    const int M = carry;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const int o = __shfl_xor(cmax, off);
        cmax = o > cmax ? o : cmax;
    }
    if (lane == 0 && cmax > 0) atomicMax(&cmax_s, cmax);
    if (tid == 0) pre[a.R] = M;

    const uint64_t* regq = a.regions + (int64_t)q * a.rc;  // region w at regq + w*nq*rc
    // When the previous best and the whole pass fit the buffer at once, both
    // go straight to LDS with direct-to-LDS dword loads (lane l of a wave
    // instruction writes dword l after the instruction's base; lanes past a
    // region's end are masked off), every region's in the same round: no
    // registers hold them and no load waits for another.  Wave w takes
    // regions w, w + NW, ...; 64 dwords (32 entries) per instruction.
    const bool direct = M <= LCAP - fill && M >= 4 * a.R;  // dense regions (sparse ones: one round below)
    if (direct) {
        __syncthreads();  // pre[] complete
        const uint32_t lb = __builtin_amdgcn_readfirstlane(
            (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)smem);
        const uint32_t* bsrc = (const uint32_t*)(a.best + (int64_t)q * k);
        for (int o = 64 * wave; o < 2 * fill; o += 64 * NW)
            if (o + lane < 2 * fill) lds_load4(bsrc + o + lane, __builtin_amdgcn_readfirstlane(lb + 4 * o));
        for (int w = wave; w < a.R; w += NW) {
            const int p0 = __builtin_amdgcn_readfirstlane(pre[w]);
            const int c2 = 2 * (__builtin_amdgcn_readfirstlane(pre[w + 1]) - p0);
            const uint32_t* src = (const uint32_t*)(regq + (int64_t)w * a.nq * a.rc);
            const uint32_t dst = lb + 8 * (uint32_t)(fill + p0);
            for (int o = 0; o < c2; o += 64)
                if (o + lane < c2) lds_load4(src + o + lane, __builtin_amdgcn_readfirstlane(dst + 4 * o));
        }
        // the loads are invisible to the compiler's wait counting: every wave
        // retires its own, then the barrier publishes all of them
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
        for (int i = tid; i < fill; i += NT) buf[i] = a.best[(int64_t)q * k + i];
    }
    __syncthreads();
    // regions holding 4 to 64 entries on average and at most: gather region
    // by region (sparser regions take fewer rounds of loads entry by entry)
    const bool by_region = a.uniform == 0 && cmax_s <= 64 && M >= 4 * a.R;

    // keep the best k of buf[0..fill): the radix prefix, then a block-wide
    // append of the kept keys to the front; the smallest kept key is the
    // k-th best so far
    auto compact = [&]() {
        if (tid == 0) {
            wpos = 0;
            minkey = ~0ull;
        }
        uint64_t prefix, pmask;
        block_radix_prefix(buf, fill, k, rs, prefix, pmask);  // its barriers publish wpos/minkey
        uint64_t v[KPT];
        uint32_t keep = 0;
        uint64_t lo = ~0ull;
#pragma unroll
        for (int j = 0; j < KPT; j++) {
            const int i = tid + NT * j;
            v[j] = i < fill ? buf[i] : 0ull;
            if (i < fill && (v[j] & pmask) >= prefix) {
                keep |= 1u << j;
                lo = v[j] < lo ? v[j] : lo;
            }
        }
        int pos = wave_append(__popc(keep), &wpos);
        __syncthreads();  // every read of buf is done before the first write
#pragma unroll
        for (int j = 0; j < KPT; j++)
            if (keep & (1u << j)) buf[pos++] = v[j];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const uint64_t t = __shfl_xor(lo, off);
            lo = t < lo ? t : lo;
        }
        if ((tid & 63) == 0 && lo != ~0ull) atomicMin(&minkey, (unsigned long long)lo);
        __syncthreads();
        fill = k;
    };

    const float qmax = PM == 1 ? a.qconst[q].a : 0.0f;
    if (PM == 2) {
        // the query's E16 digit planes, read by every rescoring below
        const int words = a.d / 4;
        for (int i = tid; i < words; i += NT) {
            qh_s[i] = ((const int*)(a.qhi + (int64_t)q * a.d))[i];
            ql_s[i] = ((const int*)(a.qlo + (int64_t)q * a.d))[i];
        }
        __syncthreads();
    }
    const QConst kq = PM == 2 ? a.qconst[q] : QConst{0.0f, 0.0f, 0.0f, 0.0f};

    // Shadow pairs get their exact q4 score, one pair per thread: the row's
    // nb <= 12 blocks and scales are loaded at once, then summed against the
    // query planes and folded by the contract's fma chain in block order.
    // e[i] holds raw pairs, or pre-score keys (pkeys) after pruning.
    auto rescore = [&](uint64_t* e, int cnt, bool pkeys) {
        const int nb = a.d / 32, hb = a.d / 2;
        for (int i = tid; i < cnt; i += NT) {
            // the query planes are re-read from LDS for every pair (kept in
            // registers they would take 192 of them)
            asm volatile("" ::: "memory");
            const uint64_t v = e[i];
            const uint32_t row = pkeys ? key_index(v) : (uint32_t)v;
            const v4i* prow = (const v4i*)(a.q4codes + (int64_t)row * hb);
            const uint16_t* srow = a.q4scales + (int64_t)row * nb;
            v4i w[12];
            uint16_t sb[12];
#pragma unroll
            for (int b = 0; b < 12; b++)
                if (b < nb) w[b] = prow[b];
            if ((nb & 3) == 0) {
                // four scales per 8-byte load (a row's scales start 8-byte aligned)
#pragma unroll
                for (int b = 0; b < 12; b += 4) {
                    if (b < nb) {
                        const uint2 u = *(const uint2*)(srow + b);
                        sb[b] = (uint16_t)u.x, sb[b + 1] = (uint16_t)(u.x >> 16);
                        sb[b + 2] = (uint16_t)u.y, sb[b + 3] = (uint16_t)(u.y >> 16);
                    }
                }
            } else {
#pragma unroll
                for (int b = 0; b < 12; b++)
                    if (b < nb) sb[b] = srow[b];
            }
            const float dn = a.op == OP_COSINE ? a.dnorm[row] : 0.0f;
            const float d2 = a.op == OP_L2 ? a.dd[row] : 0.0f;
            float dotf = 0.0f;
#pragma unroll
            for (int b = 0; b < 12; b++)
                if (b < nb) dotf = __fmaf_rn(h2f(sb[b]), (float)q4_block_acc(w[b], qh_s + 8 * b, ql_s + 8 * b), dotf);
            e[i] = make_key(q4_finish_op(a.op, dotf, kq, dn, d2), row, a.smallest);
        }
    };
    // all of a pass's shadow pairs fit: rank them by pre-score first
    const bool prune = PM == 2 && M > k && M <= LCAP - fill;

    bool compacted = false;  // a compaction left the k-th best key in minkey
    for (int base = 0; base < M;) {
        const int take = (M - base) < (LCAP - fill) ? (M - base) : (LCAP - fill);
        int added = take;  // keys this batch leaves in buf (fewer after pruning)
        if (direct) {
            // the pass's entries are in place: pairs become keys there
            if (PM == 1 || (PM == 2 && prune)) {
                for (int i = tid; i < take; i += NT) {
                    const uint64_t x = buf[fill + i];
                    buf[fill + i] = PM == 1 ? dot_pair_key(x, qmax, a.smallest)
                                            : make_key(__uint_as_float((uint32_t)(x >> 32)), (uint32_t)x, a.smallest);
                }
            }
        } else if (by_region) {
            // Wave w takes regions w, w + NW, ...; lane l moves entry l of
            // each, 8 regions' loads in flight at once.  Entries outside the
            // batch [base, base + take) stay for a later batch.
            for (int w0 = wave; w0 < a.R; w0 += 8 * NW) {
                uint64_t v[8];
                int dst[8];
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const int w = w0 + t * NW;
                    dst[t] = -1;
                    v[t] = 0;
                    if (w < a.R) {
                        const int g = pre[w] + lane;
                        if (g < pre[w + 1] && g >= base && g < base + take) {
                            dst[t] = fill + (g - base);
                            v[t] = regq[(int64_t)w * a.nq * a.rc + lane];
                        }
                    }
                }
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    if (dst[t] < 0) continue;
                    uint64_t x = v[t];
                    if (PM == 1) x = dot_pair_key(x, qmax, a.smallest);
                    if (PM == 2 && prune) x = make_key(__uint_as_float((uint32_t)(x >> 32)), (uint32_t)x, a.smallest);
                    buf[dst[t]] = x;
                }
            }
        } else {
        // batches of 8 independent loads per thread keep many in flight
        for (int j0 = 0; j0 < take; j0 += 8 * NT) {
            uint64_t v[8];
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const int j = j0 + t * NT + tid;
                v[t] = 0;
                if (j < take) {
                    const int g = base + j;
                    int lo = 0, off;  // last region w with pre[w] <= g, g's place in it
                    if (a.uniform > 0) {
                        lo = g / a.uniform;
                        off = g - lo * a.uniform;
                    } else {
                        int hi = a.R;
                        while (hi - lo > 1) {
                            const int mid = (lo + hi) >> 1;
                            if (pre[mid] <= g) lo = mid;
                            else hi = mid;
                        }
                        off = g - pre[lo];
                    }
                    v[t] = regq[(int64_t)lo * a.nq * a.rc + off];
                    if (PM == 1) v[t] = dot_pair_key(v[t], qmax, a.smallest);
                }
            }
            if (PM == 2 && prune) {
#pragma unroll
                for (int t = 0; t < 8; t++)
                    v[t] = make_key(__uint_as_float((uint32_t)(v[t] >> 32)), (uint32_t)v[t], a.smallest);
            }
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const int j = j0 + t * NT + tid;
                if (j < take) buf[fill + j] = v[t];
            }
        }
        }
        __syncthreads();
        if (PM == 2) {
            if (prune) {
                // Two stages.  The k pairs with the best pre-scores are
                // rescored first; with the old best keys they give a k-th
                // best exact key tk that the new k-th best can only exceed.
                // A pair's exact score is within the margin of its pre-score,
                // so of the other pairs only those passing shadow_bound(tk)
                // (the scan's own threshold test) can still make the best k.
                uint64_t prefix, pmask;
                block_radix_prefix(buf + fill, take, k, rs, prefix, pmask);
                // best-k pairs to the front, the rest after them
                if (tid == 0) wpos = 0, wpos2 = 0;
                uint64_t v[KPT];
                uint32_t inT = 0, inR = 0;
#pragma unroll
                for (int j = 0; j < KPT; j++) {
                    const int i = tid + NT * j;
                    v[j] = i < take ? buf[fill + i] : 0ull;
                    if (i < take) {
                        if ((v[j] & pmask) >= prefix) inT |= 1u << j;
                        else inR |= 1u << j;
                    }
                }
                __syncthreads();  // counters set, every read of buf done
                int pt = wave_append(__popc(inT), &wpos);
                int pr = wave_append(__popc(inR), &wpos2);
#pragma unroll
                for (int j = 0; j < KPT; j++) {
                    if (inT & (1u << j)) buf[fill + pt++] = v[j];
                    if (inR & (1u << j)) buf[fill + k + pr++] = v[j];
                }
                __syncthreads();
                const int nr = wpos2;
                rescore(buf + fill, k, true);
                __syncthreads();
                // k-th best exact key of the old best and the rescored k
                if (tid == 0) minkey = ~0ull;
                uint64_t lo = ~0ull;
                if (fill > 0) {
                    block_radix_prefix(buf, fill + k, k, rs, prefix, pmask);
                    for (int i = tid; i < fill + k; i += NT) {
                        const uint64_t key = buf[i];
                        if ((key & pmask) >= prefix) lo = key < lo ? key : lo;
                    }
                } else {
                    __syncthreads();
                    for (int i = tid; i < k; i += NT) lo = buf[fill + i] < lo ? buf[fill + i] : lo;
                }
#pragma unroll
                for (int off = 32; off >= 1; off >>= 1) {
                    const uint64_t t = __shfl_xor(lo, off);
                    lo = t < lo ? t : lo;
                }
                if (lane == 0 && lo != ~0ull) atomicMin(&minkey, (unsigned long long)lo);
                __syncthreads();
                const float lbv = shadow_bound(minkey, a.qbound[2 * q], a.qbound[2 * q + 1], a.smallest);
                // the other pairs within that bound, packed after the k
                if (tid == 0) wpos = 0;
                uint32_t keep = 0;
#pragma unroll
                for (int j = 0; j < KPT; j++) {
                    const int i = tid + NT * j;
                    v[j] = i < nr ? buf[fill + k + i] : 0ull;
                    const float p = key_score(v[j], a.smallest);
                    if (i < nr && (a.smallest ? p <= lbv : p >= lbv)) keep |= 1u << j;
                }
                __syncthreads();
                int pos = wave_append(__popc(keep), &wpos);
#pragma unroll
                for (int j = 0; j < KPT; j++)
                    if (keep & (1u << j)) buf[fill + k + pos++] = v[j];
                __syncthreads();
                added = k + wpos;
                rescore(buf + fill + k, wpos, true);
                __syncthreads();
            } else {
                rescore(buf + fill, added, false);
                __syncthreads();
            }
        }
        fill += added;
        base += take;
        if (fill > k && (fill == LCAP || base == M)) {
            compact();
            compacted = true;
        }
    }
    if (fill > k) {
        compact();
        compacted = true;
    }
    // threshold for the next pass: the k-th key once k keys exist
    if (fill == k && !compacted) {
        // exactly k keys arrived: their minimum (rare; no compaction ran)
        if (tid == 0) minkey = ~0ull;
        __syncthreads();
        uint64_t lo = ~0ull;
        for (int i = tid; i < fill; i += NT) lo = buf[i] < lo ? buf[i] : lo;
        if (lo != ~0ull) atomicMin(&minkey, (unsigned long long)lo);
        __syncthreads();
    }
    const uint64_t kth = fill == k ? (uint64_t)minkey : 0ull;
    if (a.out_ids && a.unsorted && fill == k) {
        // final pass for a caller that re-sorts (the reference finish): the
        // kept keys in buffer order, except that the k-th best goes last, so
        // position k-1 still holds the worst kept score
        for (int i = tid; i < fill; i += NT)
            if (buf[i] == kth) kpos = i;
        __syncthreads();
        const int p = kpos;
        for (int i = tid; i < k; i += NT) {
            const uint64_t key = buf[i == k - 1 ? p : (i == p ? k - 1 : i)];
            a.out_ids[(int64_t)q * k + i] = (int32_t)key_index(key);
            if (a.out_scores) a.out_scores[(int64_t)q * k + i] = key_score(key, a.smallest);
        }
    } else if (a.out_ids) {
        // final pass: ids and scores in (value, index) order
        const int S = next_pow2(fill < 2 ? 2 : fill);
        for (int i = fill + tid; i < S; i += NT) buf[i] = 0;
        __syncthreads();
        block_sort_desc_regs<NT>(buf, S);
        for (int i = tid; i < k; i += NT) {
            const uint64_t key = i < fill ? buf[i] : 0ull;
            a.out_ids[(int64_t)q * k + i] = key ? (int32_t)key_index(key) : -1;
            if (a.out_scores) a.out_scores[(int64_t)q * k + i] = key ? key_score(key, a.smallest) : 0.0f;
        }
    } else {
        // intermediate pass: the best keys in any order, and the threshold
        for (int i = tid; i < fill; i += NT) a.best[(int64_t)q * k + i] = buf[i];
    }
    if (tid == 0) {
        a.bcnt[q] = fill;
        a.tau[q] = kth;
    }
}

// ----------------------------------------------------------------- hosts

// Register budget: NA*KS*4 VGPRs of resident A fragments plus the staged
// chunk (4 VGPRs per 16-byte load per thread) must leave room for the
// accumulators and the epilogue at two waves per SIMD.
static constexpr bool mq_valid(int na, int wq, int ks) {
    return (na == 2 && wq == 4 && ks <= 12) || (na == 1 && wq == 4) || (na == 2 && wq == 1 && ks <= 4) ||
           (na == 1 && wq == 2 && ks >= 8);
}

MqShape mq_shape(int op, int ks, int64_t nq) {
    MqShape s;
    s.ks = ks;
    const int qpb = op == OP_DOT ? 32 : 16;
    if (nq >= 8 * qpb && ks <= 12) {
        s.na = 2, s.wq = 4;
    } else if (nq >= 4 * qpb) {
        s.na = 1, s.wq = 4;
    } else if (ks <= 4) {
        s.na = 2, s.wq = 1;
    } else {
        s.na = 1, s.wq = 2;
    }
    s.qg = s.wq * s.na * qpb;
    s.chunk = (4 / s.wq) * 32;
    const int segs = (s.chunk * (ks * 32 + 16) + 1023) / 1024;
    s.tile = ((segs + 3) / 4) * 4 * 1024;
    const int narr = (op == OP_DOT || op == OP_DOT16) ? 1 : 2;
    const int ctile = ((narr * ((s.chunk + 63) / 64) + 3) / 4) * 4 * 256;
    const int vpw = s.tile / 4096 + ctile / 1024;
    s.tile_bytes = mq_nbuf(s.tile + ctile, vpw) * (s.tile + ctile);  // chunk tiles + row constants
    return s;
}

bool mq_supported_ks(int ks) { return ks == 2 || ks == 4 || ks == 8 || ks == 12 || ks == 16; }

template <int OP, int ENC, int NA, int WQ, int MODE, bool SMALL, int KS>
static hipError_t launch_mq_one(const MqArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    if constexpr (mq_valid(NA, WQ, KS)) {
        hipLaunchKernelGGL((mq_scan_kernel<OP, ENC, KS, NA, WQ, MODE, SMALL>), grid, dim3(256), lds, s, a);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

template <int OP, int ENC, int NA, int WQ, int MODE, bool SMALL>
static hipError_t launch_mq_ks(const MqArgs& a, int ks, dim3 grid, size_t lds, hipStream_t s) {
    switch (ks) {
        case 2: return launch_mq_one<OP, ENC, NA, WQ, MODE, SMALL, 2>(a, grid, lds, s);
        case 4: return launch_mq_one<OP, ENC, NA, WQ, MODE, SMALL, 4>(a, grid, lds, s);
        case 8: return launch_mq_one<OP, ENC, NA, WQ, MODE, SMALL, 8>(a, grid, lds, s);
        case 12: return launch_mq_one<OP, ENC, NA, WQ, MODE, SMALL, 12>(a, grid, lds, s);
        case 16: return launch_mq_one<OP, ENC, NA, WQ, MODE, SMALL, 16>(a, grid, lds, s);
        default: return hipErrorInvalidValue;
    }
}

template <int OP, int ENC, int NA, int WQ>
static hipError_t launch_mq_mode(const MqArgs& a, int ks, dim3 grid, size_t lds, hipStream_t s) {
    if (a.out_scores) return launch_mq_ks<OP, ENC, NA, WQ, MQ_SCORES, false>(a, ks, grid, lds, s);
    if (a.smallest) return launch_mq_ks<OP, ENC, NA, WQ, MQ_APPEND, true>(a, ks, grid, lds, s);
    return launch_mq_ks<OP, ENC, NA, WQ, MQ_APPEND, false>(a, ks, grid, lds, s);
}

template <int OP, int ENC>
static hipError_t launch_mq_op(const MqShape& sh, const MqArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    if (sh.na == 2 && sh.wq == 4) return launch_mq_mode<OP, ENC, 2, 4>(a, sh.ks, grid, lds, s);
    if (sh.na == 1 && sh.wq == 4) return launch_mq_mode<OP, ENC, 1, 4>(a, sh.ks, grid, lds, s);
    if (sh.na == 2 && sh.wq == 1) return launch_mq_mode<OP, ENC, 2, 1>(a, sh.ks, grid, lds, s);
    if (sh.na == 1 && sh.wq == 2) return launch_mq_mode<OP, ENC, 1, 2>(a, sh.ks, grid, lds, s);
    return hipErrorInvalidValue;
}

hipError_t launch_mq_scan(int op, const MqShape& sh, const MqArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    if (op == OP_DOT) return launch_mq_op<OP_DOT, MQ_E8>(sh, a, grid, lds, s);
    if (op == OP_DOT16) return launch_mq_op<OP_DOT16, MQ_E16>(sh, a, grid, lds, s);
    if (op == OP_COSINE) return launch_mq_op<OP_COSINE, MQ_E16>(sh, a, grid, lds, s);
    return launch_mq_op<OP_L2, MQ_E16>(sh, a, grid, lds, s);
}

// Threads of the select kernel: 1024 (16K-key buffer) when a pass is
// expected to leave more keys than the 256-thread, 4K-key buffer holds.
int mq_select_threads(int64_t expect_keys) { return expect_keys > 4096 ? 1024 : 256; }

size_t mq_select_lds(int threads, int R) { return (size_t)threads * 16 * 8 + (size_t)(R + 1) * 4; }

template <int PM>
static void launch_mq_select_pm(const MqSelectArgs& a, int threads, size_t lds, hipStream_t s) {
    if constexpr (PM != 2) {
        if (threads == 1024) {
            hipLaunchKernelGGL((mq_select_kernel<1024, PM>), dim3((unsigned)a.nq), dim3(1024), lds, s, a);
            return;
        }
    }
    if (threads == 512)
        hipLaunchKernelGGL((mq_select_kernel<512, PM>), dim3((unsigned)a.nq), dim3(512), lds, s, a);
    else
        hipLaunchKernelGGL((mq_select_kernel<256, PM>), dim3((unsigned)a.nq), dim3(256), lds, s, a);
}

hipError_t launch_mq_select(const MqSelectArgs& a, int threads, hipStream_t s) {
    const size_t lds = mq_select_lds(threads, a.R);
    // shadow pairs: rows of at most 12 blocks (a row's blocks are in flight
    // per thread)
    if (a.pairs == 2 && (a.d % 32 != 0 || a.d > 384)) return hipErrorInvalidValue;
    // shadow pairs: at most 512 threads (the rescoring's registers at 1024
    // threads spill)
    if (a.pairs == 2 && threads > 512) return hipErrorInvalidValue;
    if (threads != 256 && threads != 512 && threads != 1024) return hipErrorInvalidValue;
    if (a.pairs == 1)
        launch_mq_select_pm<1>(a, threads, lds, s);
    else if (a.pairs == 2)
        launch_mq_select_pm<2>(a, threads, lds, s);
    else
        launch_mq_select_pm<0>(a, threads, lds, s);
    return hipGetLastError();
}

}  // namespace manta
