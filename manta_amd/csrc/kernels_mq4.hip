// kernels_mq4.hip -- many queries against one shared q4 candidate matrix
// (rows of NB blocks: 32 nibbles and an f16 scale per block) on the i8
// matrix cores of gfx950.
//
// The q4 score is a per-block integer dot product folded into f32 by an fma
// chain over the blocks (a_b = sum nib*code16 exact; dotf = fma(s_b, a_b,
// dotf) for b = 0..NB-1; qd = dotf*qs), so every block needs its own exact
// sum.  One v_mfma_i32_32x32x32_i8 covers exactly one block (K = 32) for 16
// queries x {hi, lo} E16 digit (A rows [hi q0-7 | lo q0-7 | hi q8-15 |
// lo q8-15], resident in VGPRs) against 32 candidates.  Each lane reads the
// 8 nibble bytes of its half block from LDS and widens them in two ALU ops
// per dword to bytes holding 16*nibble: (x << 4) & 0xF0F0F0F0 gives the even
// elements, x & 0xF0F0F0F0 the odd ones, which is the element order the
// query planes are encoded in.  Both digit sums are then 16x the true ones,
// a16 = (hi << 8) + lo = 16*a_b is exact in int32 and in f32 (a multiple of
// 16 below 2^27), and fma(s_b/16, f32(a16), dotf) equals the contract's
// fma(s_b, a_b, dotf) bit for bit (same exact product, same addend).
//
// Chunks, passes, regions, compaction and the select are those of the q8
// multi-query path (kernels_mq.hip).
#include "mq_common.hpp"

namespace manta {

// Pre-score bound of a q4 query: every op works on E16 codes, so dot
// compares qd (the score itself) with the loosened threshold.
template <int OP>
__device__ __forceinline__ float mq4_bound(uint64_t tk, const QConst& qc, bool smallest) {
    if (OP != OP_DOT) return mq_bound<OP>(tk, qc, smallest);
    if (!tk) return smallest ? __builtin_inff() : -__builtin_inff();
    const float ts = key_score(tk, smallest);
    return smallest ? loosen_up(ts) : loosen_down(ts);
}

template <int OP, int NB, int NA, int WQ, int MODE, bool SMALL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void mq_q4_kernel(MqArgs a) {
    constexpr int PITCH = NB * 16;            // packed bytes per candidate row
    constexpr int D = NB * 32;                // elements per row (query plane width)
    constexpr int P = PITCH + 16;             // LDS row pitch
    constexpr int WR = 4 / WQ;                // waves splitting the rows of a chunk
    constexpr int CHUNK = WR * 32;            // rows per chunk (one 32-row block per wave)
    constexpr int SEGS = (CHUNK * P + 1023) / 1024;
    constexpr int DPW = (SEGS + 3) / 4;       // 16-byte direct-to-LDS loads per wave per chunk
    constexpr int TILE = DPW * 4 * 1024;
    // per-row constants: NB f16 block scales, then |d| (cosine) or |d|^2 (l2)
    constexpr int SCB = CHUNK * NB * 2;                     // block-scale bytes per chunk
    constexpr int SCSEG = (SCB + 255) / 256;                // 256-byte segments
    constexpr int RCSEG = OP == OP_DOT ? 0 : (CHUNK + 63) / 64;
    constexpr int CPW = (SCSEG + RCSEG + 3) / 4;            // 4-byte loads per wave per chunk
    constexpr int CTILE = CPW * 4 * 256;
    constexpr int VPW = DPW + CPW;
    constexpr int NBUF = mq_nbuf(TILE + CTILE, VPW);
    constexpr int QPB = 16;                   // queries per A block (E16)
    constexpr int QPW = NA * QPB;
    constexpr int QG = WQ * QPW;
    constexpr int QPL = 8;                    // queries per lane per A block
    constexpr int NFW = (QG + 63) / 64;
    constexpr bool APPEND = MODE == MQ_APPEND;

    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* tiles = smem;                                   // [NBUF][TILE]
    uint8_t* consts = smem + NBUF * TILE;                    // [NBUF][CTILE]
    uint64_t* scratch_extra = (uint64_t*)(smem + NBUF * (TILE + CTILE));
    __shared__ uint64_t tau_s[QG];
    __shared__ __attribute__((aligned(16))) float bnd_s[QG];
    __shared__ __attribute__((aligned(16))) float qa_s[QG];   // QConst.a = qs
    __shared__ __attribute__((aligned(16))) float qc_s[QG];   // QConst.c = |q|^2
    __shared__ int cnt_s[QG];
    __shared__ uint64_t flags[2][NFW];
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

    for (int i = tid; i < QG; i += 256) {
        const int q = q0 + i;
        const bool ok = q < a.nq;
        const QConst qc = ok ? a.qconst[q] : QConst{1.0f, 0.0f, 0.0f, 0.0f};
        qa_s[i] = qc.a;
        qc_s[i] = qc.c;
        const uint64_t tk = (APPEND && ok) ? a.tau[q] : 0ull;
        tau_s[i] = ok ? tk : ~0ull;
        bnd_s[i] = ok ? mq4_bound<OP>(tk, qc, SMALL) : (SMALL ? -__builtin_inff() : __builtin_inff());
        cnt_s[i] = 0;
    }

    // ---- A operand: E16 digit planes (q4 nibble order), one K step per block
    v4i av[NA][NB];
#pragma unroll
    for (int na = 0; na < NA; na++) {
        const int i = lane & 31;
        const int blk = i >> 3;  // 0: hi q0-7, 1: lo q0-7, 2: hi q8-15, 3: lo q8-15
        const int q = q0 + wq * QPW + na * 16 + (blk >> 1) * 8 + (i & 7);
        const int8_t* plane = (blk & 1) ? a.qlo : a.qhi;
        const bool ok = q < a.nq;
        const int8_t* src = plane + (int64_t)(ok ? q : 0) * D + half * 16;
#pragma unroll
        for (int b = 0; b < NB; b++) av[na][b] = ok ? *(const v4i*)(src + b * 32) : v4i{0, 0, 0, 0};
    }

    // slot u (0..7) of A block na: hi accumulator r, lo r+4, and its query
    auto slot_r = [](int u) { return u < 4 ? u : u + 4; };
    auto slot_lq = [&](int na, int u) { return wq * QPW + na * QPB + 8 * (u >> 2) + 4 * half + (u & 3); };
    uint32_t live[NA];
#pragma unroll
    for (int na = 0; na < NA; na++) {
        live[na] = 0;
#pragma unroll
        for (int u = 0; u < QPL; u++)
            if (q0 + slot_lq(na, u) < a.nq) live[na] |= 1u << u;
    }

    uint64_t* wreg = a.regions + (int64_t)blockIdx.x * a.nq * a.rc;
    const int64_t r0 = a.row_begin + (int64_t)blockIdx.x * a.rows_per_wg;
    int64_t r1 = r0 + a.rows_per_wg;
    if (r1 > a.row_end) r1 = a.row_end;

    const int wave_s = __builtin_amdgcn_readfirstlane(wave);
    const uint8_t* sc_bytes = (const uint8_t*)a.scales;
    const float* rowc_src = OP == OP_COSINE ? a.dnorm : a.dd;
    auto issue_chunk = [&](int64_t c0, int buf) {
        const int8_t* base = a.codes + c0 * PITCH;
        const int left = (int)(r1 - c0 < CHUNK ? r1 - c0 : CHUNK);
        const int lim = left * PITCH - 16;
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
        const uint8_t* sbase = sc_bytes + c0 * (NB * 2);
        const int slim = left * NB * 2 - 4;
#pragma unroll
        for (int i = 0; i < CPW; i++) {
            const int cs = wave_s * CPW + i;  // segments past SCSEG + RCSEG are filler
            if (cs >= SCSEG && cs < SCSEG + RCSEG) {
                const int row = (cs - SCSEG) * 64 + lane;
                lds_load4(rowc_src + c0 + (row < left ? row : left - 1), ct + cs * 256);
            } else {
                const int o = (cs < SCSEG ? cs : 0) * 256 + lane * 4;
                lds_load4(sbase + (o < slim ? o : slim), ct + cs * 256);
            }
        }
    };
    __syncthreads();
    __builtin_amdgcn_s_waitcnt(0);  // retire the A loads where the compiler sees it (see kernels_mq.hip)
#pragma unroll
    for (int j = 0; j < NBUF - 1; j++)
        if (r0 + j * CHUNK < r1) issue_chunk(r0 + j * CHUNK, j);

    // One 32-row block: per q4 block an MFMA and the fma into dotf.  Block
    // b+1's MFMA is issued before block b's fmas, so two accumulator sets are
    // in flight.  Empty volatile asm statements (kept in program order) pin
    // that schedule: block b's fmas complete before the dotf fence, and block
    // b+2's B fragment -- hence its MFMA -- comes after it.
    auto multiply = [&](const uint8_t* tile, const uint8_t* ctile, float (&dotf)[NA][QPL]) {
        const uint8_t* bp = tile + (wr * 32 + (lane & 31)) * P + half * 8;
        const uint16_t* sp = (const uint16_t*)ctile + (wr * 32 + (lane & 31)) * NB;
        auto widen = [&](int b) {
            const uint2 nb2 = *(const uint2*)(bp + b * 16);
            v4i bf = {(int)((nb2.x << 4) & 0xF0F0F0F0u), (int)(nb2.x & 0xF0F0F0F0u),
                      (int)((nb2.y << 4) & 0xF0F0F0F0u), (int)(nb2.y & 0xF0F0F0F0u)};
            asm volatile("" : "+v"(bf));
            return bf;
        };
#pragma unroll
        for (int na = 0; na < NA; na++)
#pragma unroll
            for (int u = 0; u < QPL; u++) dotf[na][u] = 0.0f;
        v16i accn[NA];
        {
            const v4i bf = widen(0);
#pragma unroll
            for (int na = 0; na < NA; na++) accn[na] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[na][0], bf, v16i{}, 0, 0, 0);
        }
#pragma unroll
        for (int b = 0; b < NB; b++) {
            v16i acc[NA];
#pragma unroll
            for (int na = 0; na < NA; na++) acc[na] = accn[na];
            if (b + 1 < NB) {
                const v4i bf = widen(b + 1);
#pragma unroll
                for (int na = 0; na < NA; na++)
                    accn[na] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[na][b + 1], bf, v16i{}, 0, 0, 0);
            }
            const float s16 = fmul_rn(h2f(sp[b]), 0.0625f);  // exact: a power-of-two scaling
#pragma unroll
            for (int na = 0; na < NA; na++) {
#pragma unroll
                for (int u = 0; u < QPL; u++) {
                    const int r = slot_r(u);
                    const int a16 = (acc[na][r] << 8) + acc[na][r + 4];
                    dotf[na][u] = __fmaf_rn(s16, (float)a16, dotf[na][u]);
                }
            }
#pragma unroll
            for (int na = 0; na < NA; na++)
#pragma unroll
                for (int u = 0; u < QPL; u++) asm volatile("" : "+v"(dotf[na][u]));
        }
    };

    struct SlotVals {
        float bq[QPL], qa[QPL], qcv[QPL];
    };
    auto slot_vals = [&](int na, SlotVals& v) {
        const int lq0 = wq * QPW + na * QPB + 4 * half;
#pragma unroll
        for (int m = 0; m < QPL / 4; m++) {
            const float4 b4 = *(const float4*)&bnd_s[lq0 + 8 * m];
            v.bq[4 * m] = b4.x, v.bq[4 * m + 1] = b4.y, v.bq[4 * m + 2] = b4.z, v.bq[4 * m + 3] = b4.w;
            const float4 a4 = *(const float4*)&qa_s[lq0 + 8 * m];
            v.qa[4 * m] = a4.x, v.qa[4 * m + 1] = a4.y, v.qa[4 * m + 2] = a4.z, v.qa[4 * m + 3] = a4.w;
            if (OP == OP_L2) {
                const float4 c4 = *(const float4*)&qc_s[lq0 + 8 * m];
                v.qcv[4 * m] = c4.x, v.qcv[4 * m + 1] = c4.y, v.qcv[4 * m + 2] = c4.z, v.qcv[4 * m + 3] = c4.w;
            }
        }
    };
    // pre-scores: qd = dotf*qs (dot: the score; cosine: q.d), l2: dist^2
    auto pre_of = [&](float dotf, const SlotVals& v, int u, float rowc) {
        const float qd = fmul_rn(dotf, v.qa[u]);
        return OP == OP_L2 ? fsub_rn(fadd_rn(v.qcv[u], rowc), fmul_rn(2.0f, qd)) : qd;
    };
    auto keep_of = [&](const SlotVals& v, int u, float p, float rowc) {
        const float bv = OP == OP_COSINE ? fmul_rn(v.bq[u], rowc) : v.bq[u];
        return SMALL ? !(p > bv) : !(p < bv);
    };
    auto score_of = [&](float p, int lq, float rowc) {
        if (OP == OP_DOT) return p;
        if (OP == OP_COSINE) {
            const float den = fmul_rn(a.qconst[q0 + lq].b, rowc);
            return den == 0.0f ? 0.0f : fdiv_rn(p, den);
        }
        return fsqrt_rn(p < 0.0f ? 0.0f : p);
    };

    int buf = 0, par = 0;
    for (int64_t c0 = r0; c0 < r1; c0 += CHUNK, buf = buf == NBUF - 1 ? 0 : buf + 1, par ^= 1) {
        if (APPEND) {
            for (int w = wave; w < NFW; w += 4) {
                const int i = w * 64 + lane;
                const uint64_t m = __ballot(i < QG && cnt_s[i < QG ? i : 0] > a.rc - 2 * CHUNK);
                if (lane == 0) flags[par][w] = m;
            }
        }
        mq_wait_barrier<VPW, NBUF - 2>((r1 - c0 - 1) / CHUNK);
        const int nbuf = buf == 0 ? NBUF - 1 : buf - 1;
        if (APPEND) {
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
                            bnd_s[lq] = mq4_bound<OP>(minkey, a.qconst[q0 + lq], SMALL);
                        }
                    }
                    __syncthreads();
                }
            }
        }
        if (APPEND && c0 + (NBUF - 1) * CHUNK < r1) issue_chunk(c0 + (NBUF - 1) * CHUNK, nbuf);
        const uint8_t* tile = tiles + buf * TILE;
        const uint8_t* ctile = consts + buf * CTILE;
        const int64_t row = c0 + wr * 32 + (lane & 31);
        const float rowc = OP == OP_DOT ? 0.0f : ((const float*)(ctile + SCSEG * 256))[wr * 32 + (lane & 31)];
        float dotf[NA][QPL];
        multiply(tile, ctile, dotf);
        if (row < r1) {
            if (!APPEND) {
#pragma unroll
                for (int na = 0; na < NA; na++) {
                    SlotVals v;
                    slot_vals(na, v);
#pragma unroll
                    for (int u = 0; u < QPL; u++) {
                        if (!((live[na] >> u) & 1)) continue;
                        const int lq = slot_lq(na, u);
                        a.out_scores[(int64_t)(q0 + lq) * a.n + row] = score_of(pre_of(dotf[na][u], v, u, rowc), lq, rowc);
                    }
                }
            }
        }
        if (APPEND) {
            bool any = false;
            SlotVals v[NA];
#pragma unroll
            for (int na = 0; na < NA; na++) {
                slot_vals(na, v[na]);
#pragma unroll
                for (int u = 0; u < QPL; u++) any |= keep_of(v[na], u, pre_of(dotf[na][u], v[na], u, rowc), rowc);
            }
            if (__ballot(any && row < r1) && row < r1) {
#pragma unroll
                for (int na = 0; na < NA; na++) {
#pragma unroll
                    for (int u = 0; u < QPL; u++) {
                        const float p = pre_of(dotf[na][u], v[na], u, rowc);
                        if (keep_of(v[na], u, p, rowc)) {
                            const int lq = slot_lq(na, u);
                            const uint64_t key = make_key(score_of(p, lq, rowc), (uint32_t)row, SMALL);
                            if (key > tau_s[lq]) {
                                const int pos = atomicAdd(&cnt_s[lq], 1);
                                wreg[(uint32_t)((q0 + lq) * a.rc + pos)] = key;
                            }
                        }
                    }
                }
            }
        }
        if (!APPEND && c0 + (NBUF - 1) * CHUNK < r1) issue_chunk(c0 + (NBUF - 1) * CHUNK, nbuf);
    }
    if (!APPEND) return;
    __syncthreads();
    for (int i = tid; i < QG; i += 256)
        if (q0 + i < a.nq) a.counts[(int64_t)blockIdx.x * a.nq + q0 + i] = cnt_s[i];
}

// ----------------------------------------------------------------- hosts

static constexpr bool mq4_valid(int na, int wq, int nb) {
    return (na == 2 && wq == 4 && nb <= 12) || (na == 1 && wq == 4) || (na == 2 && wq == 1 && nb <= 4) ||
           (na == 1 && wq == 2 && nb >= 8);
}

MqShape mq4_shape(int op, int nb, int64_t nq) {
    (void)op;
    MqShape s;
    s.ks = nb;
    if (nq >= 128 && nb <= 12) {
        s.na = 2, s.wq = 4;
    } else if (nq >= 64) {
        s.na = 1, s.wq = 4;
    } else if (nb <= 4) {
        s.na = 2, s.wq = 1;
    } else {
        s.na = 1, s.wq = 2;
    }
    s.qg = s.wq * s.na * 16;
    s.chunk = (4 / s.wq) * 32;
    const int segs = (s.chunk * (nb * 16 + 16) + 1023) / 1024;
    s.tile = ((segs + 3) / 4) * 4 * 1024;
    const int scseg = (s.chunk * nb * 2 + 255) / 256;
    const int rcseg = op == OP_DOT ? 0 : (s.chunk + 63) / 64;
    const int ctile = ((scseg + rcseg + 3) / 4) * 4 * 256;
    const int vpw = s.tile / 4096 + ctile / 1024;
    s.tile_bytes = mq_nbuf(s.tile + ctile, vpw) * (s.tile + ctile);
    return s;
}

bool mq4_supported_nb(int nb) { return nb == 1 || nb == 2 || nb == 4 || nb == 8 || nb == 12 || nb == 16; }

template <int OP, int NA, int WQ, int MODE, bool SMALL, int NB>
static hipError_t launch_mq4_one(const MqArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    if constexpr (mq4_valid(NA, WQ, NB)) {
        hipLaunchKernelGGL((mq_q4_kernel<OP, NB, NA, WQ, MODE, SMALL>), grid, dim3(256), lds, s, a);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

template <int OP, int NA, int WQ, int MODE, bool SMALL>
static hipError_t launch_mq4_nb(const MqArgs& a, int nb, dim3 grid, size_t lds, hipStream_t s) {
    switch (nb) {
        case 1: return launch_mq4_one<OP, NA, WQ, MODE, SMALL, 1>(a, grid, lds, s);
        case 2: return launch_mq4_one<OP, NA, WQ, MODE, SMALL, 2>(a, grid, lds, s);
        case 4: return launch_mq4_one<OP, NA, WQ, MODE, SMALL, 4>(a, grid, lds, s);
        case 8: return launch_mq4_one<OP, NA, WQ, MODE, SMALL, 8>(a, grid, lds, s);
        case 12: return launch_mq4_one<OP, NA, WQ, MODE, SMALL, 12>(a, grid, lds, s);
        case 16: return launch_mq4_one<OP, NA, WQ, MODE, SMALL, 16>(a, grid, lds, s);
        default: return hipErrorInvalidValue;
    }
}

template <int OP, int NA, int WQ>
static hipError_t launch_mq4_mode(const MqArgs& a, int nb, dim3 grid, size_t lds, hipStream_t s) {
    if (a.out_scores) return launch_mq4_nb<OP, NA, WQ, MQ_SCORES, false>(a, nb, grid, lds, s);
    if (a.smallest) return launch_mq4_nb<OP, NA, WQ, MQ_APPEND, true>(a, nb, grid, lds, s);
    return launch_mq4_nb<OP, NA, WQ, MQ_APPEND, false>(a, nb, grid, lds, s);
}

template <int OP>
static hipError_t launch_mq4_op(const MqShape& sh, const MqArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    if (sh.na == 2 && sh.wq == 4) return launch_mq4_mode<OP, 2, 4>(a, sh.ks, grid, lds, s);
    if (sh.na == 1 && sh.wq == 4) return launch_mq4_mode<OP, 1, 4>(a, sh.ks, grid, lds, s);
    if (sh.na == 2 && sh.wq == 1) return launch_mq4_mode<OP, 2, 1>(a, sh.ks, grid, lds, s);
    if (sh.na == 1 && sh.wq == 2) return launch_mq4_mode<OP, 1, 2>(a, sh.ks, grid, lds, s);
    return hipErrorInvalidValue;
}

hipError_t launch_mq4_scan(int op, const MqShape& sh, const MqArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    if (op == OP_DOT) return launch_mq4_op<OP_DOT>(sh, a, grid, lds, s);
    if (op == OP_COSINE) return launch_mq4_op<OP_COSINE>(sh, a, grid, lds, s);
    return launch_mq4_op<OP_L2>(sh, a, grid, lds, s);
}

}  // namespace manta
