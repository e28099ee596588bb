// kernels_embed.hip -- the embed pipeline on gfx950:
//   gather(table, tokens) -> @matmul(proj) -> masked mean_pool -> normalize
// (reference steps: gatherTensor tensor_ops.go:751-979, matmulTensor
// :981-1062, meanPoolMaskedTensor :1210-1275, normalizeRows :1114-1138).
//
// GEMM core: 64 x 128 output tile per workgroup (4 waves, each 32 x 64 =
// two 32x32 MFMA tiles), K staged through LDS in chunks of 64 with
// v_mfma_f32_32x32x16_f16 (f32 accumulate).  The A tile is either a plain
// f16 matrix or rows gathered straight from the embedding table by token id
// (the [B,T,D] gather never reaches HBM).  The projection chunk is written
// to LDS transposed (n-major, k contiguous) so both MFMA operands are single
// 16-byte LDS reads; a q8 projection is widened int8 -> f16 exactly and its
// per-column scale applied in the epilogue.  In pooled mode the epilogue
// sums the masked rows of its tile per column and writes one partial per
// (sequence, row tile); a finalize kernel adds the partials in a fixed
// order, divides by the count and L2-normalizes.
#include <algorithm>

#include "device_common.hpp"
#include "kernels.hpp"

namespace manta {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int EM = 64;       // rows per tile
constexpr int EN = 128;      // columns per tile
constexpr int EK = 64;       // K per LDS chunk
constexpr int LDA = EK + 8;  // halfs per LDS row (pad against bank conflicts)
constexpr int LDB = EK + 8;


template <bool GATHER, bool Q8B, bool POOL>
__global__ __launch_bounds__(256) void embed_gemm_kernel(EmbedArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 As[EM * LDA];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[EN * LDB];
    __shared__ float red[2][EN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1;  // 32-row half of the tile
    const int wn = wave & 1;   // 64-column half of the tile
    const int n0 = blockIdx.y * EN;

    // Row tile -> (sequence, first position) in pooled/gather mode, else m0.
    int64_t seq = 0, t0 = 0, m0 = 0;
    if (POOL) {
        seq = blockIdx.x / a.tiles_per_seq;
        t0 = (int64_t)(blockIdx.x % a.tiles_per_seq) * EM;
    } else {
        m0 = (int64_t)blockIdx.x * EM;
    }

    // Each thread stages two 16-byte A segments per chunk: rows r0 and r0+32.
    const int seg_col = tid & 7;  // 16-byte column within the 128-byte chunk row
    const int r0 = tid >> 3;      // 0..31
    const _Float16* arow[2];
    bool arow_live[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int r = r0 + h * 32;
        arow[h] = nullptr;
        arow_live[h] = false;
        if (POOL) {
            const int64_t t = t0 + r;
            if (t < a.T) {
                const int64_t pos = seq * a.T + t;
                int idx = a.tokens[pos];
                if (idx < 0 || idx >= a.vocab) {
                    report_gather_error(a.err, pos, idx);
                } else if (!a.mask || a.mask[pos] != 0) {
                    arow[h] = (const _Float16*)a.table + (int64_t)idx * a.K;
                    arow_live[h] = true;
                }
            }
        } else {
            const int64_t m = m0 + r;
            if (m < a.M) {
                if (GATHER) {
                    int idx = a.tokens[m];
                    if (idx < 0 || idx >= a.vocab) {
                        report_gather_error(a.err, m, idx);
                    } else {
                        arow[h] = (const _Float16*)a.table + (int64_t)idx * a.K;
                        arow_live[h] = true;
                    }
                } else {
                    arow[h] = (const _Float16*)a.A + m * a.K;
                    arow_live[h] = true;
                }
            }
        }
    }

    f16v acc[2];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;

    for (int k0 = 0; k0 < a.K; k0 += EK) {
        // ---- stage A: 64 rows x 64 k
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int k = k0 + seg_col * 8;
            h8 v = (h8)(_Float16)0.0f;
            if (arow_live[h] && k < a.K) v = *(const h8*)(arow[h] + k);
            *(h8*)&As[(r0 + h * 32) * LDA + seg_col * 8] = v;
        }
        // ---- stage B transposed: Bs[n][k]
        if (!Q8B) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int u = tid + 256 * j;
                const int kg = u >> 6;   // 0..7: k group of 8
                const int np = u & 63;   // pair of columns
                const int n = n0 + 2 * np;
                h8 c0, c1;
#pragma unroll
                for (int kk = 0; kk < 8; kk++) {
                    const int k = k0 + kg * 8 + kk;
                    uint32_t w = 0;
                    if (k < a.K && n < a.N) w = *(const uint32_t*)((const uint16_t*)a.B + (int64_t)k * a.N + n);
                    c0[kk] = __builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
                    c1[kk] = __builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
                }
                *(h8*)&Bs[(2 * np) * LDB + kg * 8] = c0;
                *(h8*)&Bs[(2 * np + 1) * LDB + kg * 8] = c1;
            }
        } else {
            const int kg = tid >> 5;  // 0..7
            const int nq = tid & 31;  // quad of columns
            const int n = n0 + 4 * nq;
            h8 c[4];
#pragma unroll
            for (int kk = 0; kk < 8; kk++) {
                const int k = k0 + kg * 8 + kk;
                uint32_t w = 0;
                if (k < a.K && n < a.N) w = *(const uint32_t*)((const int8_t*)a.B + (int64_t)k * a.N + n);
#pragma unroll
                for (int q = 0; q < 4; q++) c[q][kk] = (_Float16)(int)(int8_t)((w >> (8 * q)) & 0xFF);
            }
#pragma unroll
            for (int q = 0; q < 4; q++) *(h8*)&Bs[(4 * nq + q) * LDB + kg * 8] = c[q];
        }
        __syncthreads();
        // ---- 4 MFMA k-steps of 16
#pragma unroll
        for (int s = 0; s < EK / 16; s++) {
            const int kofs = s * 16 + (lane >> 5) * 8;
            h8 av = *(const h8*)&As[(wm * 32 + (lane & 31)) * LDA + kofs];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                h8 bv = *(const h8*)&Bs[(wn * 64 + t * 32 + (lane & 31)) * LDB + kofs];
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc[t], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    // Output element (tile t, acc r): row 8*(r/4) + 4*(lane/32) + r%4 of the
    // wave's 32 rows, column lane%32 of the tile.
    if (!POOL) {
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int n = n0 + wn * 64 + t * 32 + (lane & 31);
            if (n >= a.N) continue;
            const float cs = Q8B ? a.colscale[n] : 1.0f;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = m0 + wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < a.M) a.Y[m * a.N + n] = Q8B ? acc[t][r] * cs : acc[t][r];
            }
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < 2; t++) {
        float s = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int64_t tt = t0 + wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            bool live = tt < a.T && (!a.mask || a.mask[seq * a.T + tt] != 0);
            if (live) s += acc[t][r];
        }
        s += __shfl_xor(s, 32);
        if (lane < 32) red[wm][wn * 64 + t * 32 + lane] = s;
    }
    __syncthreads();
    if (tid < EN) {
        const int n = n0 + tid;
        if (n < a.N) {
            float v = red[0][tid] + red[1][tid];
            if (Q8B) v *= a.colscale[n];
            a.P[((int64_t)seq * a.tiles_per_seq + (blockIdx.x % a.tiles_per_seq)) * a.N + n] = v;
        }
    }
}

// ------------------------------------------------ pipelined GEMM (K%32, N%128)

// Direct-to-LDS loads (gfx950): each lane's 16 bytes land at M0 + 16*lane.
__device__ __forceinline__ void eg_lds_load16(const void* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}

// vmcnt(J*L) + barrier while at least J chunks were issued after the current
// one, else the next smaller J (a smaller count only waits longer).
template <int L, int J>
__device__ __forceinline__ void eg_wait_barrier(int after) {
    if constexpr (J <= 0) {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    } else {
        if (after >= J)
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(J * L) : "memory");
        else
            eg_wait_barrier<L, J - 1>(after);
    }
}

// Bt[n][k] = B[k][n] as f16 (a q8 projection widened exactly; its column
// scale is applied in the GEMM epilogue), so both MFMA operands are rows.
__global__ void embed_transpose_b_kernel(const void* __restrict__ B, int q8, int K, int N,
                                         uint16_t* __restrict__ Bt) {
    __shared__ uint16_t t[32][33];
    const int k0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int r = ty; r < 32; r += 8) {
        const int k = k0 + r, n = n0 + tx;
        uint16_t v = 0;
        if (k < K && n < N)
            v = q8 ? f2h((float)((const int8_t*)B)[(int64_t)k * N + n]) : ((const uint16_t*)B)[(int64_t)k * N + n];
        t[r][tx] = v;
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int n = n0 + r, k = k0 + tx;
        if (n < N && k < K) Bt[(int64_t)n * K + k] = t[tx][r];
    }
}

// Workgroup: 4 waves stacked in M, each a 64-row tile (pooled mode: 64
// positions of one sequence) x 128 columns, as 2 x 4 tiles of
// v_mfma_f32_32x32x16_f16.  K moves in chunks of 32 through a 3-stage ring
// of LDS buffers filled by direct-to-LDS loads (A rows gathered by token id
// straight from the table); each 64-byte LDS row stores its 16-byte column c
// at c ^ ((row >> 2) & 3), so the 32 lanes reading one column of 32 rows
// spread over the banks.  Rows past the tile's range, masked or with a bad
// token id read row 0 and are left out of the store or the pool.
constexpr int EG_WM = 64, EG_WN = 128, EG_KC = 32, EG_NST = 3;
constexpr int EG_AST = 4 * EG_WM * EG_KC * 2;  // A bytes per stage (256 rows)
constexpr int EG_BST = EG_WN * EG_KC * 2;      // B bytes per stage
constexpr int EG_STAGE = EG_AST + EG_BST;

template <bool GATHER, bool Q8B, bool POOL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void embed_gemm2_kernel(EmbedArgs a,
                                                                                                 const uint16_t* Bt) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n0 = blockIdx.y * EG_WN;
    const int64_t tile = (int64_t)blockIdx.x * 4 + wave;
    const int64_t ntiles = POOL ? a.batches * a.tiles_per_seq : (a.M + EG_WM - 1) / EG_WM;
    int64_t seq = 0, t0 = 0, m0 = 0;
    if (POOL) {
        seq = tile / a.tiles_per_seq;
        t0 = (tile % a.tiles_per_seq) * EG_WM;
    } else {
        m0 = tile * EG_WM;
    }

    // source rows of this lane's 4 A segments: rows 16 s + lane/4 of the tile
    const uint8_t* arow[4];
#pragma unroll
    for (int sg = 0; sg < 4; sg++) {
        const int r = sg * 16 + (lane >> 2);
        int64_t src = 0;  // row of the table (gather) or of A
        if (tile < ntiles) {
            if (POOL) {
                const int64_t t = t0 + r;
                if (t < a.T) {
                    const int idx = a.tokens[seq * a.T + t];
                    if (idx >= 0 && idx < a.vocab) src = idx;
                    else report_gather_error(a.err, seq * a.T + t, idx);
                }
            } else {
                const int64_t m = m0 + r;
                if (m < a.M) {
                    if (GATHER) {
                        const int idx = a.tokens[m];
                        if (idx >= 0 && idx < a.vocab) src = idx;
                        else report_gather_error(a.err, m, idx);
                    } else {
                        src = m;
                    }
                }
            }
        }
        const int c = (lane & 3) ^ ((r >> 2) & 3);  // global 16-byte column of the stored one
        arow[sg] = (const uint8_t*)(GATHER ? a.table : a.A) + src * a.K * 2 + c * 16;
    }
    const uint8_t* brow[2];
#pragma unroll
    for (int sg = 0; sg < 2; sg++) {
        const int n = (wave * 2 + sg) * 16 + (lane >> 2);
        const int c = (lane & 3) ^ ((n >> 2) & 3);
        brow[sg] = (const uint8_t*)Bt + (int64_t)(n0 + n) * a.K * 2 + c * 16;
    }
    const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)smem);
    auto issue = [&](int kc, int st) {
        const uint32_t sa = __builtin_amdgcn_readfirstlane(base + st * EG_STAGE + wave * 4 * 1024);
#pragma unroll
        for (int sg = 0; sg < 4; sg++) eg_lds_load16(arow[sg] + kc * EG_KC * 2, sa + sg * 1024);
        const uint32_t sb = __builtin_amdgcn_readfirstlane(base + st * EG_STAGE + EG_AST + wave * 2 * 1024);
#pragma unroll
        for (int sg = 0; sg < 2; sg++) eg_lds_load16(brow[sg] + kc * EG_KC * 2, sb + sg * 1024);
    };
    const int nk = a.K / EG_KC;
#pragma unroll
    for (int st = 0; st < EG_NST - 1; st++)
        if (st < nk) issue(st, st);

    f16v acc[2][4];
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int cb = 0; cb < 4; cb++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[rb][cb][r] = 0.0f;

    const int l32 = lane & 31, hf = lane >> 5;
    int st = 0;
    for (int kc = 0; kc < nk; kc++, st = st == EG_NST - 1 ? 0 : st + 1) {
        eg_wait_barrier<6, EG_NST - 2>(nk - 1 - kc);
        if (kc + EG_NST - 1 < nk) issue(kc + EG_NST - 1, st == 0 ? EG_NST - 1 : st - 1);
        const uint8_t* As = smem + st * EG_STAGE + wave * EG_WM * EG_KC * 2;
        const uint8_t* Bs = smem + st * EG_STAGE + EG_AST;
#pragma unroll
        for (int ks = 0; ks < EG_KC / 16; ks++) {
            const int c = ks * 2 + hf;  // 16-byte column of this lane's 8 k
            h8 av[2], bv[4];
#pragma unroll
            for (int rb = 0; rb < 2; rb++) {
                const int r = rb * 32 + l32;
                av[rb] = *(const h8*)(As + r * 64 + ((c ^ ((r >> 2) & 3)) * 16));
            }
#pragma unroll
            for (int cb = 0; cb < 4; cb++) {
                const int n = cb * 32 + l32;
                bv[cb] = *(const h8*)(Bs + n * 64 + ((c ^ ((n >> 2) & 3)) * 16));
            }
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
#pragma unroll
                for (int cb = 0; cb < 4; cb++)
                    acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[rb], bv[cb], acc[rb][cb], 0, 0, 0);
        }
    }
    if (tile >= ntiles) return;

    // Output element (rb, cb, r): row rb*32 + 8*(r/4) + 4*(lane/32) + r%4 of
    // the wave's tile, column cb*32 + lane%32.
    if (!POOL) {
#pragma unroll
        for (int cb = 0; cb < 4; cb++) {
            const int n = n0 + cb * 32 + l32;
            const float cs = Q8B ? a.colscale[n] : 1.0f;
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int64_t m = m0 + rb * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
                    if (m >= a.M) continue;
                    const float v = Q8B ? acc[rb][cb][r] * cs : acc[rb][cb][r];
                    if (a.Y16) a.Y16[m * a.N + n] = f2h(a.gelu ? gelu_value_f32(v) : v);
                    else a.Y[m * a.N + n] = v;
                }
        }
        return;
    }
    bool live[2][16];
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int64_t t = t0 + rb * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
            live[rb][r] = t < a.T && (!a.mask || a.mask[seq * a.T + t] != 0);
        }
#pragma unroll
    for (int cb = 0; cb < 4; cb++) {
        float sum = 0.0f;
#pragma unroll
        for (int rb = 0; rb < 2; rb++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                if (live[rb][r]) sum += acc[rb][cb][r];
        sum += __shfl_xor(sum, 32);
        const int n = n0 + cb * 32 + l32;
        if (hf == 0) {
            if (Q8B) sum *= a.colscale[n];
            a.P[(seq * a.tiles_per_seq + t0 / EG_WM) * a.N + n] = sum;
        }
    }
}

// Sum the row-tile partials of one sequence in order, divide by the number
// of unmasked positions (count 0 -> zeros), L2-normalize (f64 sum of
// squares, f32 norm, zero norm leaves the row unchanged) and round to f16.
__global__ __launch_bounds__(256) void embed_finalize_kernel(const float* __restrict__ P, int tiles,
                                                             const int32_t* __restrict__ mask,
                                                             int64_t T, int N, uint16_t* __restrict__ out) {
    __shared__ float row[4096];
    __shared__ double red[256];
    __shared__ int cnt_red[256];
    const int64_t b = blockIdx.x;
    const int tid = threadIdx.x;
    int cnt = 0;
    for (int64_t t = tid; t < T; t += 256) cnt += (!mask || mask[b * T + t] != 0) ? 1 : 0;
    cnt_red[tid] = cnt;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s) cnt_red[tid] += cnt_red[tid + s];
        __syncthreads();
    }
    const int count = cnt_red[0];
    const float inv = count ? 1.0f / (float)count : 0.0f;
    double ss = 0.0;
    for (int c = tid; c < N; c += 256) {
        float v = 0.0f;
        for (int s = 0; s < tiles; s++) v += P[(b * tiles + s) * N + c];
        v = count ? v * inv : 0.0f;
        row[c] = v;
        ss += (double)v * (double)v;
    }
    red[tid] = ss;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s) red[tid] += red[tid + s];
        __syncthreads();
    }
    const float norm = (float)__builtin_sqrt(red[0]);
    for (int c = tid; c < N; c += 256) {
        float v = row[c];
        if (norm != 0.0f) v = v / norm;
        out[b * N + c] = f2h(v);
    }
}

// gatherTensor rank-2 table x indices: one 16-byte (or 2-byte tail) copy per
// thread; an out-of-range index leaves a zero row and is reported.
__global__ void gather_rows_f16_kernel(const uint16_t* __restrict__ table, int64_t vocab, int64_t d,
                                       const int32_t* __restrict__ idx, int64_t nidx,
                                       uint16_t* __restrict__ out, unsigned long long* err) {
    const int64_t row = blockIdx.x;
    const int id = idx[row];
    const bool ok = id >= 0 && id < vocab;
    if (!ok && threadIdx.x == 0) report_gather_error(err, row, id);
    for (int64_t c = threadIdx.x; c < d; c += blockDim.x)
        out[row * d + c] = ok ? table[(int64_t)id * d + c] : (uint16_t)0;
}

// meanPoolMaskedTensor rank 3: one thread per (b, c), positions summed in
// order, then multiplied by 1/float(count) -- the reference's exact order.
__global__ void mean_pool_masked_kernel(const float* __restrict__ x, const int32_t* __restrict__ mask,
                                        int64_t B, int64_t T, int64_t C, float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B * C) return;
    const int64_t b = i / C, c = i % C;
    float s = 0.0f;
    int64_t count = 0;
    for (int64_t t = 0; t < T; t++) {
        if (mask[b * T + t] == 0) continue;
        count++;
        s += x[(b * T + t) * C + c];
    }
    if (count) s *= 1.0f / (float)count;
    out[i] = count ? s : 0.0f;
}

// normalizeRows: one thread per row, f64 sum of squares in column order,
// f32 norm, f32 division; zero rows unchanged -- the reference's order.
__global__ void normalize_rows_kernel(float* __restrict__ x, int64_t rows, int64_t cols) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    float* p = x + r * cols;
    double s = 0.0;
    for (int64_t c = 0; c < cols; c++) {
        double v = (double)p[c];
        s = __dadd_rn(s, __dmul_rn(v, v));
    }
    const float norm = (float)__builtin_sqrt(s);
    if (norm == 0.0f) return;
    for (int64_t c = 0; c < cols; c++) p[c] = fdiv_rn(p[c], norm);
}

// ----------------------------------------------------------------- hosts

// ------------------------------------- single-pass GEMM (f16 B, N = 384)
//
// Workgroup = one 32-row tile x all 384 columns: 4 waves of 96 columns,
// each three 32x32 tiles of v_mfma_f32_32x32x16_f16.  K moves in chunks of
// 32 through a 5-stage ring of LDS buffers filled by direct-to-LDS loads:
// the A chunk (32 rows x 64 bytes, rows gathered by token id) by 4-byte
// loads, the projection chunk (32 k-rows x 768 bytes, row-major as stored)
// by 16-byte loads.  The projection's MFMA operand (8 consecutive k of one
// column per lane) comes from two ds_read_tr16_b64: lane i of a 16-lane
// group receives element i%4 of the 8 bytes that lane 4j + i/4 of the group
// addresses, j = 0..3, so a group addresses 4 k-rows x 16 columns and lane
// i gets column i at those 4 k.  A projection row stores its 16-byte chunk
// c at c ^ 2*(k%4), so the 4 rows a group reads hit distinct banks; an A row
// stores its 16-byte column c at c ^ ((row >> 2) & 3) as in the pipelined
// kernel.
constexpr int E3_WM = 32, E3_N = 384, E3_KC = 32, E3_NST = 5;
constexpr int E3_AST = E3_WM * E3_KC * 2;  // A bytes per stage (2 KB)
constexpr int E3_BST = E3_KC * E3_N * 2;   // projection bytes per stage (24 KB)
constexpr int E3_STAGE = E3_AST + E3_BST;

__device__ __forceinline__ void eg_lds_load4(const void* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}

typedef short v4s __attribute__((ext_vector_type(4)));

// ds_read_tr16_b64 at an LDS byte address given as a generic pointer
__device__ __forceinline__ v4s lds_read_tr16(const uint8_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)p);
}

template <bool GATHER, bool POOL>
__global__ __launch_bounds__(256) void embed_gemm3_kernel(EmbedArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ float rowv[E3_N];
    __shared__ double dred[4];
    __shared__ int ired[4];
    __shared__ int last;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t tile = blockIdx.x;
    int64_t seq = 0, t0 = 0, m0 = 0;
    if (POOL) {
        seq = tile / a.tiles_per_seq;
        t0 = (tile % a.tiles_per_seq) * E3_WM;
    } else {
        m0 = tile * E3_WM;
    }
    const int K = a.K;

    // A loads: this wave's two 256-byte pieces of a stage (rows 4L .. 4L+3,
    // L = 2*wave + u); lane i fills stored dword i%16 of row 4L + i/16.
    const uint8_t* asrc[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int r = 4 * (2 * wave + u) + (lane >> 4);
        int64_t src = 0;
        if (POOL) {
            const int64_t t = t0 + r;
            if (t < a.T) {
                const int idx = a.tokens[seq * a.T + t];
                if (idx >= 0 && idx < a.vocab) src = idx;
                else report_gather_error(a.err, seq * a.T + t, idx);
            }
        } else {
            const int64_t m = m0 + r;
            if (m < a.M) {
                if (GATHER) {
                    const int idx = a.tokens[m];
                    if (idx >= 0 && idx < a.vocab) src = idx;
                    else report_gather_error(a.err, m, idx);
                } else {
                    src = m;
                }
            }
        }
        const int c = ((lane & 15) >> 2) ^ ((r >> 2) & 3);
        asrc[u] = (const uint8_t*)(GATHER ? a.table : a.A) + src * K * 2 + c * 16 + (lane & 3) * 4;
    }
    // projection loads: this wave's six 1 KB pieces of a stage
    int boff[6];
#pragma unroll
    for (int u = 0; u < 6; u++) {
        const int x = (6 * wave + u) * 1024 + lane * 16;
        const int kr = x / (E3_N * 2);
        const int c = ((x % (E3_N * 2)) / 16) ^ (2 * (kr & 3));
        boff[u] = kr * E3_N * 2 + c * 16;
    }
    const uint8_t* bsrc = (const uint8_t*)a.B;
    const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)smem);
    // Workgroups walk the K chunks from different starting points, so the
    // CUs do not all ask L2 for the same projection lines at once.
    const int nk = K / E3_KC;
    const int rot = (int)(tile % nk);
    auto issue = [&](int kci, int st) {
        const int kc = kci + rot < nk ? kci + rot : kci + rot - nk;
        const uint32_t sa = __builtin_amdgcn_readfirstlane(base + st * E3_STAGE + wave * 2 * 256);
#pragma unroll
        for (int u = 0; u < 2; u++) eg_lds_load4(asrc[u] + kc * E3_KC * 2, sa + u * 256);
        const uint32_t sb = __builtin_amdgcn_readfirstlane(base + st * E3_STAGE + E3_AST + wave * 6 * 1024);
        const uint8_t* bk = bsrc + (int64_t)kc * E3_KC * E3_N * 2;
#pragma unroll
        for (int u = 0; u < 6; u++) eg_lds_load16(bk + boff[u], sb + u * 1024);
    };
#pragma unroll
    for (int st = 0; st < E3_NST - 1; st++)
        if (st < nk) issue(st, st);

    // transpose-read offsets of this lane's projection operands: group G =
    // lane/16 takes k-half G>>1 and 16-column half G&1 of a 32-column tile;
    // lane s of the group addresses k-row s/4, columns 4*(s%4) .. +3
    const int G = lane >> 4, s16 = lane & 15;
    const int trow = (8 * (G >> 1) + (s16 >> 2)) * E3_N * 2 + 8 * (s16 & 1);
    int tcol[3];
#pragma unroll
    for (int cb = 0; cb < 3; cb++) {
        const int c = (wave * 96 + cb * 32 + 16 * (G & 1)) / 8 + ((s16 & 3) >> 1);
        tcol[cb] = (c ^ (2 * (s16 >> 2))) * 16;
    }

    f16v acc[3];
#pragma unroll
    for (int cb = 0; cb < 3; cb++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[cb][r] = 0.0f;

    const int l32 = lane & 31, hf = lane >> 5;
    int st = 0;
    for (int kc = 0; kc < nk; kc++, st = st == E3_NST - 1 ? 0 : st + 1) {
        eg_wait_barrier<8, E3_NST - 2>(nk - 1 - kc);
        if (kc + E3_NST - 1 < nk) issue(kc + E3_NST - 1, st == 0 ? E3_NST - 1 : st - 1);
        const uint8_t* As = smem + st * E3_STAGE;
        const uint8_t* Bs = As + E3_AST;
#pragma unroll
        for (int ks = 0; ks < E3_KC / 16; ks++) {
            const int c = ks * 2 + hf;
            const h8 av = *(const h8*)(As + l32 * 64 + ((c ^ ((l32 >> 2) & 3)) * 16));
#pragma unroll
            for (int cb = 0; cb < 3; cb++) {
                const uint8_t* p = Bs + trow + tcol[cb] + ks * 16 * E3_N * 2;
                // k 0..3 of the lane's 8, then k 4..7 (four k-rows further)
                const v4s lo = lds_read_tr16(p);
                const v4s hi = lds_read_tr16(p + 4 * E3_N * 2);
                const h8 bv = __builtin_bit_cast(h8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                acc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc[cb], 0, 0, 0);
            }
        }
    }

    // Output element (cb, r): row 8*(r/4) + 4*(lane/32) + r%4 of the tile,
    // column wave*96 + cb*32 + lane%32.
    if (!POOL) {
#pragma unroll
        for (int cb = 0; cb < 3; cb++) {
            const int n = wave * 96 + cb * 32 + l32;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = m0 + 8 * (r >> 2) + 4 * hf + (r & 3);
                if (m < a.M) a.Y[m * E3_N + n] = acc[cb][r];
            }
        }
        return;
    }
    bool live[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int64_t t = t0 + 8 * (r >> 2) + 4 * hf + (r & 3);
        live[r] = t < a.T && (!a.mask || a.mask[seq * a.T + t] != 0);
    }
    // publish the tile's column sums (agent-scope stores, then the ticket)
    unsigned int* pdst = (unsigned int*)(a.P + (seq * a.tiles_per_seq + t0 / E3_WM) * E3_N);
#pragma unroll
    for (int cb = 0; cb < 3; cb++) {
        float sum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r++)
            if (live[r]) sum += acc[cb][r];
        sum += __shfl_xor(sum, 32);
        if (hf == 0)
            __hip_atomic_store(pdst + wave * 96 + cb * 32 + l32, __float_as_uint(sum), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    // publication order as finish_wave_lists (kernels_score.hip): agent-scope
    // atomic stores retired by s_waitcnt vmcnt(0), barrier, then the ticket
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(&a.tickets[seq], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (unsigned)(a.tiles_per_seq - 1);
    __syncthreads();
    if (!last) return;
    // the sequence's embedding: partials added in tile order, divided by the
    // count of unmasked positions, L2-normalized (as embed_finalize_kernel)
    int cnt = 0;
    for (int64_t t = tid; t < a.T; t += 256) cnt += (!a.mask || a.mask[seq * a.T + t] != 0) ? 1 : 0;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) cnt += __shfl_xor(cnt, off);
    if (lane == 0) ired[wave] = cnt;
    __syncthreads();
    const int count = ired[0] + ired[1] + ired[2] + ired[3];
    const float inv = count ? 1.0f / (float)count : 0.0f;
    const unsigned int* psrc = (const unsigned int*)(a.P + seq * a.tiles_per_seq * E3_N);
    double ss = 0.0;
    for (int c = tid; c < E3_N; c += 256) {
        // 8 tiles' partials in flight at a time, added in tile order
        float v = 0.0f;
        for (int s0 = 0; s0 < a.tiles_per_seq; s0 += 8) {
            unsigned int pv[8];
#pragma unroll
            for (int u = 0; u < 8; u++)
                pv[u] = s0 + u < a.tiles_per_seq
                            ? __hip_atomic_load(psrc + (s0 + u) * E3_N + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                            : 0u;
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (s0 + u < a.tiles_per_seq) v += __uint_as_float(pv[u]);
        }
        v = count ? v * inv : 0.0f;
        rowv[c] = v;
        ss += (double)v * (double)v;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    if (lane == 0) dred[wave] = ss;
    __syncthreads();
    const float norm = (float)__builtin_sqrt(dred[0] + dred[1] + dred[2] + dred[3]);
    for (int c = tid; c < E3_N; c += 256) {
        float v = rowv[c];
        if (norm != 0.0f) v = v / norm;
        a.out[seq * E3_N + c] = f2h(v);
    }
    if (tid == 0) __hip_atomic_store(&a.tickets[seq], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Pooled embed, 128-row x 96-column workgroup tiles (4 waves of 32 rows,
// each three 32x32 tiles): a workgroup reads a quarter of the projection and
// 128 gathered rows per K pass, about half the bytes of a 32-row x 384-column
// tile, which at C1's size is what bounds the K loop.  Same K ring (A by
// 16-byte loads, projection rows by 4-byte loads, unswizzled: rows 192 bytes
// apart put the 4 k-rows of a transpose read on distinct banks), same
// publication and last-tile finish as embed_gemm3_kernel (partials of the 4
// column slices of a row tile side by side).
constexpr int E4_WM = 128, E4_WN = 96, E4_NST = 6;
constexpr int E4_AST = E4_WM * E3_KC * 2;   // 8 KB
constexpr int E4_BST = E3_KC * E4_WN * 2;   // 6 KB
constexpr int E4_STAGE = E4_AST + E4_BST;

__global__ __launch_bounds__(256) void embed_gemm4_kernel(EmbedArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ float rowv[E3_N];
    __shared__ float colw[4][E4_WN];
    __shared__ double dred[4];
    __shared__ int ired[4];
    __shared__ int last;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t tile = blockIdx.x;
    const int slice = blockIdx.y;
    const int nb0 = slice * E4_WN;
    const int64_t seq = tile / a.tiles_per_seq;
    const int64_t t0 = (tile % a.tiles_per_seq) * E4_WM;
    const int K = a.K;

    // A loads: this wave's 32 rows, two 1 KB loads of 16 rows; lane i fills
    // stored column i%4 of row 16u + i/4
    const uint8_t* asrc[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int r = 32 * wave + 16 * u + (lane >> 2);
        int64_t src = 0;
        const int64_t t = t0 + r;
        if (t < a.T) {
            const int idx = a.tokens[seq * a.T + t];
            if (idx >= 0 && idx < a.vocab) src = idx;
            else report_gather_error(a.err, seq * a.T + t, idx);
        }
        const int c = (lane & 3) ^ ((r >> 2) & 3);
        asrc[u] = (const uint8_t*)a.table + src * K * 2 + c * 16;
    }
    // projection loads: six 256-byte pieces of the stage per wave
    int boff[6];
#pragma unroll
    for (int v = 0; v < 6; v++) {
        const int x = (6 * wave + v) * 256 + lane * 4;
        boff[v] = (x / (E4_WN * 2)) * E3_N * 2 + nb0 * 2 + x % (E4_WN * 2);
    }
    const uint8_t* bsrc = (const uint8_t*)a.B;
    const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)smem);
    const int nk = K / E3_KC;
    const int rot = (int)((tile * 4 + slice) % nk);
    auto issue = [&](int kci, int st) {
        const int kc = kci + rot < nk ? kci + rot : kci + rot - nk;
        const uint32_t sa = __builtin_amdgcn_readfirstlane(base + st * E4_STAGE + wave * 2 * 1024);
#pragma unroll
        for (int u = 0; u < 2; u++) eg_lds_load16(asrc[u] + kc * E3_KC * 2, sa + u * 1024);
        const uint32_t sb = __builtin_amdgcn_readfirstlane(base + st * E4_STAGE + E4_AST + wave * 6 * 256);
        const uint8_t* bk = bsrc + (int64_t)kc * E3_KC * E3_N * 2;
#pragma unroll
        for (int v = 0; v < 6; v++) eg_lds_load4(bk + boff[v], sb + v * 256);
    };
#pragma unroll
    for (int st = 0; st < E4_NST - 1; st++)
        if (st < nk) issue(st, st);

    const int G = lane >> 4, s16 = lane & 15;
    const int trow = (8 * (G >> 1) + (s16 >> 2)) * E4_WN * 2;
    const int tcol = (16 * (G & 1) + 4 * (s16 & 3)) * 2;

    f16v acc[3];
#pragma unroll
    for (int cb = 0; cb < 3; cb++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[cb][r] = 0.0f;

    const int l32 = lane & 31, hf = lane >> 5;
    int st = 0;
    for (int kc = 0; kc < nk; kc++, st = st == E4_NST - 1 ? 0 : st + 1) {
        eg_wait_barrier<8, E4_NST - 2>(nk - 1 - kc);
        if (kc + E4_NST - 1 < nk) issue(kc + E4_NST - 1, st == 0 ? E4_NST - 1 : st - 1);
        const uint8_t* As = smem + st * E4_STAGE + wave * 32 * 64;
        const uint8_t* Bs = smem + st * E4_STAGE + E4_AST;
#pragma unroll
        for (int ks = 0; ks < E3_KC / 16; ks++) {
            const int c = ks * 2 + hf;
            const h8 av = *(const h8*)(As + l32 * 64 + ((c ^ ((l32 >> 2) & 3)) * 16));
#pragma unroll
            for (int cb = 0; cb < 3; cb++) {
                const uint8_t* p = Bs + trow + tcol + cb * 64 + ks * 16 * E4_WN * 2;
                const v4s lo = lds_read_tr16(p);
                const v4s hi = lds_read_tr16(p + 4 * E4_WN * 2);
                const h8 bv = __builtin_bit_cast(h8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                acc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc[cb], 0, 0, 0);
            }
        }
    }

    // column sums of the wave's unmasked rows, then of the 4 waves in order
    bool live[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int64_t t = t0 + 32 * wave + 8 * (r >> 2) + 4 * hf + (r & 3);
        live[r] = t < a.T && (!a.mask || a.mask[seq * a.T + t] != 0);
    }
#pragma unroll
    for (int cb = 0; cb < 3; cb++) {
        float sum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r++)
            if (live[r]) sum += acc[cb][r];
        sum += __shfl_xor(sum, 32);
        if (hf == 0) colw[wave][cb * 32 + l32] = sum;
    }
    __syncthreads();
    unsigned int* pdst = (unsigned int*)(a.P + (seq * a.tiles_per_seq + t0 / E4_WM) * E3_N + nb0);
    if (tid < E4_WN) {
        const float v = ((colw[0][tid] + colw[1][tid]) + colw[2][tid]) + colw[3][tid];
        __hip_atomic_store(pdst + tid, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(&a.tickets[seq], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (unsigned)(4 * a.tiles_per_seq - 1);
    __syncthreads();
    if (!last) return;
    int cnt = 0;
    for (int64_t t = tid; t < a.T; t += 256) cnt += (!a.mask || a.mask[seq * a.T + t] != 0) ? 1 : 0;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) cnt += __shfl_xor(cnt, off);
    if (lane == 0) ired[wave] = cnt;
    __syncthreads();
    const int count = ired[0] + ired[1] + ired[2] + ired[3];
    const float inv = count ? 1.0f / (float)count : 0.0f;
    const unsigned int* psrc = (const unsigned int*)(a.P + seq * a.tiles_per_seq * E3_N);
    double ss = 0.0;
    for (int c = tid; c < E3_N; c += 256) {
        float v = 0.0f;
        for (int s0 = 0; s0 < a.tiles_per_seq; s0 += 8) {
            unsigned int pv[8];
#pragma unroll
            for (int u = 0; u < 8; u++)
                pv[u] = s0 + u < a.tiles_per_seq
                            ? __hip_atomic_load(psrc + (s0 + u) * E3_N + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                            : 0u;
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (s0 + u < a.tiles_per_seq) v += __uint_as_float(pv[u]);
        }
        v = count ? v * inv : 0.0f;
        rowv[c] = v;
        ss += (double)v * (double)v;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    if (lane == 0) dred[wave] = ss;
    __syncthreads();
    const float norm = (float)__builtin_sqrt(dred[0] + dred[1] + dred[2] + dred[3]);
    for (int c = tid; c < E3_N; c += 256) {
        float v = rowv[c];
        if (norm != 0.0f) v = v / norm;
        a.out[seq * E3_N + c] = f2h(v);
    }
    if (tid == 0) __hip_atomic_store(&a.tickets[seq], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

hipError_t launch_embed_gemm4(const EmbedArgs& a, hipStream_t s) {
    const size_t lds = (size_t)E4_NST * E4_STAGE;
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)embed_gemm4_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lds);
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL(embed_gemm4_kernel, dim3((unsigned)(a.batches * a.tiles_per_seq), 4u), dim3(256), lds, s, a);
    return hipGetLastError();
}

// Pooled embed for small batches (C1: 64 sequences of 128 tokens), one round
// of loads per workgroup.  Grid: 128-row tiles x 4 column slices of 96 (256
// workgroups at C1: one per CU, and workgroups that all start within about a
// microsecond -- a grid four times larger takes about 5 us just to start).
// A workgroup loads everything it multiplies at once, as its first act: the
// tokens and mask of its rows, then the 128 gathered table rows straight
// into VGPRs (a wave's 32 rows, the whole of K: K/4 registers a lane) and
// the projection slice (all K rows x 192 bytes of [K][N], read as stored)
// direct to LDS.  Table row loads are made contiguous by numbering k inside
// each 64-k block so that MFMA step s (0..3) of k-half h takes k = 32h + 8s
// + 0..7: lane (row r, half h) holds table[r][64b + 32h .. +31] for block b,
// 64 bytes, and the projection's transpose reads address the same k rows.
// The mask of the lane's row is loaded with its token, so after the MFMAs
// the pooling needs no further load (a wave ballot gives every lane the
// liveness of its 16 accumulator rows).  Each workgroup publishes its masked
// column sums (and the tile's unmasked count) to P; the last workgroup of a
// sequence adds them in tile order, pools, normalizes and writes the f16
// embedding.  (Splitting K instead of rows across the 4 waves reads the
// projection from LDS once instead of four times, but needs 351 registers a
// lane for 12 accumulator tiles and measured slower: 12.7 against 10.6 us.)
constexpr int E7_WM = 128, E7_WN = 96, E7_BROW = E7_WN * 2;

template <int NB>
__global__ __launch_bounds__(256) void embed_gemm7_kernel(EmbedArgs a, int xcd_map) {
    constexpr int K = NB * 64;
    constexpr int NBL = K * E7_BROW / 1024;  // 1 KB wave loads of the projection slice
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];  // [K][96] f16
    __shared__ float rowv[E3_N];
    __shared__ float colw[4][E7_WN];
    __shared__ double dred[4];
    __shared__ int ired[4];
    __shared__ int last;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    int64_t tile;
    int slice;
    if (xcd_map) {
        // workgroups are dealt to the 8 XCDs round robin: the 4 slices of a
        // tile go to one XCD, so the table rows one slice reads are in that
        // XCD's L2 for the other three
        const int64_t x = blockIdx.x, y = x >> 3;
        slice = (int)(y & 3);
        tile = (y >> 2) * 8 + (x & 7);
    } else {
        slice = (int)(blockIdx.x & 3);
        tile = blockIdx.x >> 2;
    }
    const int64_t seq = tile / a.tiles_per_seq;
    const int64_t t0 = (tile % a.tiles_per_seq) * E7_WM;
    const int nb0 = slice * E7_WN;

    // This lane's row (32 * wave + lane % 32 of the tile, k-half lane / 32).
    // Its token id goes first, by an asm load, then the projection slice's
    // direct-to-LDS loads (they need no token, so they travel during the
    // token's latency: 0.2 us a call on C1), then one explicit wait that
    // counts them and retires only the token (loads complete in order; a
    // compiler-placed wait could not count the asm loads and would wait for
    // all of them), then the row loads and the mask.
    const int l32 = lane & 31, hf = lane >> 5;
    int64_t src = 0;
    bool live_row = false;
    const int64_t tt = t0 + 32 * wave + l32;
    const int64_t tix = seq * a.T + (tt < a.T ? tt : a.T - 1);  // clamped in range
    int idx_raw;
    asm volatile("global_load_dword %0, %1, off" : "=v"(idx_raw) : "v"(a.tokens + tix) : "memory");
    const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)smem);
    const uint8_t* bsrc = (const uint8_t*)a.B + nb0 * 2;
    constexpr int NBW = (NBL + 3) / 4;  // projection loads of wave 0 (the others issue as many or one fewer)
    // the projection slice, rows 0 .. K-1 packed at 192 bytes (16-byte
    // pieces: a wave load covers 5 1/3 rows)
#pragma unroll
    for (int u0 = 0; u0 < NBL; u0 += 4) {
        const int u = u0 + wave;
        if (u < NBL) {
            const int x = u * 1024 + lane * 16;
            eg_lds_load16(bsrc + (int64_t)(x / E7_BROW) * E3_N * 2 + x % E7_BROW,
                          __builtin_amdgcn_readfirstlane(base + u * 1024));
        }
    }
    // the token load is older than this wave's projection loads, of which
    // all may still be outstanding (NBW, or NBW - 1 for the waves that issue
    // one fewer); idx_raw is an operand so nothing reads it before the wait
    if (NBL % 4 == 0 || wave < NBL % 4)
        asm volatile("s_waitcnt vmcnt(%1)" : "+v"(idx_raw) : "n"(NBW) : "memory");
    else
        asm volatile("s_waitcnt vmcnt(%1)" : "+v"(idx_raw) : "n"(NBW - 1 > 0 ? NBW - 1 : 0) : "memory");
    {
        if (tt < a.T) {
            const int idx = idx_raw;
            if (idx >= 0 && idx < a.vocab) src = idx;
            else if (hf == 0 && slice == 0) report_gather_error(a.err, seq * a.T + tt, idx);
        }
    }
    const uint8_t* arow = (const uint8_t*)a.table + src * K * 2 + 64 * hf;
    h8 av[NB][4];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int s = 0; s < 4; s++) av[b][s] = *(const h8*)(arow + 128 * b + 16 * s);
    if (tt < a.T) live_row = !a.mask || a.mask[seq * a.T + tt] != 0;
    // the direct-to-LDS loads are not tracked by the compiler: every wave
    // retires its own (and the row loads before them), then the barrier
    // makes all of them visible
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    // bit r of the word: row r of the wave's 32 is unmasked (both k-halves
    // of a row hold the same flag)
    const uint32_t livew = (uint32_t)__ballot(live_row);

    // MFMA step i = 4b + s; its projection fragments (one per 32-column
    // tile) are read from LDS one step ahead, so the transpose reads of step
    // i+1 are in flight under the three MFMAs of step i
    const int G = lane >> 4, s16 = lane & 15;
    const uint8_t* bt = smem + (32 * (G >> 1) + (s16 >> 2)) * E7_BROW + (16 * (G & 1) + 4 * (s16 & 3)) * 2;
    auto frag = [&](int i, int cb) {
        const uint8_t* p = bt + (64 * (i >> 2) + 8 * (i & 3)) * E7_BROW + cb * 64;
        const v4s lo = lds_read_tr16(p);
        const v4s hi = lds_read_tr16(p + 4 * E7_BROW);
        return __builtin_bit_cast(h8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    f16v acc[3];
#pragma unroll
    for (int cb = 0; cb < 3; cb++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[cb][r] = 0.0f;
    h8 bcur[3], bnext[3];
#pragma unroll
    for (int cb = 0; cb < 3; cb++) bcur[cb] = frag(0, cb);
#pragma unroll
    for (int i = 0; i < 4 * NB; i++) {
        if (i + 1 < 4 * NB) {
#pragma unroll
            for (int cb = 0; cb < 3; cb++) bnext[cb] = frag(i + 1, cb);
        }
#pragma unroll
        for (int cb = 0; cb < 3; cb++)
            acc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i >> 2][i & 3], bcur[cb], acc[cb], 0, 0, 0);
#pragma unroll
        for (int cb = 0; cb < 3; cb++) bcur[cb] = bnext[cb];
    }

    // column sums of the wave's unmasked rows (accumulator r of lane l is row
    // 8*(r/4) + 4*(l/32) + r%4), then of the 4 waves in order
#pragma unroll
    for (int cb = 0; cb < 3; cb++) {
        float sum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r++)
            if ((livew >> (8 * (r >> 2) + 4 * hf + (r & 3))) & 1u) sum += acc[cb][r];
        sum += __shfl_xor(sum, 32);
        if (hf == 0) colw[wave][cb * 32 + l32] = sum;
    }
    if (lane == 0) ired[wave] = __popc(livew);
    __syncthreads();
    const int tcount = ired[0] + ired[1] + ired[2] + ired[3];  // unmasked rows of the tile
    const int64_t ntiles = a.batches * a.tiles_per_seq;
    unsigned int* pdst = (unsigned int*)(a.P + tile * E3_N + nb0);
    unsigned int* cdst = (unsigned int*)(a.P + ntiles * E3_N);
    if (tid < E7_WN) {
        const float v = ((colw[0][tid] + colw[1][tid]) + colw[2][tid]) + colw[3][tid];
        __hip_atomic_store(pdst + tid, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid == 0 && slice == 0 && a.tiles_per_seq > 1)
        __hip_atomic_store(cdst + tile, (unsigned)tcount, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // publication order as embed_gemm4_kernel: agent-scope atomic stores
    // retired by s_waitcnt vmcnt(0), barrier, then the ticket
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(&a.tickets[seq], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (unsigned)(4 * a.tiles_per_seq - 1);
    __syncthreads();
    if (!last) return;
    // the sequence's unmasked count: this tile's own when the sequence is one
    // tile, else the published counts of its tiles
    int count = tcount;
    if (a.tiles_per_seq > 1) {
        int c = 0;
        for (int i = lane; i < a.tiles_per_seq; i += 64)
            c += (int)__hip_atomic_load(cdst + seq * a.tiles_per_seq + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) c += __shfl_xor(c, off);
        count = c;
    }
    const float inv = count ? 1.0f / (float)count : 0.0f;
    const unsigned int* psrc = (const unsigned int*)(a.P + seq * a.tiles_per_seq * E3_N);
    double ss = 0.0;
    for (int c = tid; c < E3_N; c += 256) {
        // 8 tiles' partials in flight at a time, added in tile order
        float v = 0.0f;
        for (int s0 = 0; s0 < a.tiles_per_seq; s0 += 8) {
            unsigned int pv[8];
#pragma unroll
            for (int u = 0; u < 8; u++)
                pv[u] = s0 + u < a.tiles_per_seq
                            ? __hip_atomic_load(psrc + (s0 + u) * E3_N + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                            : 0u;
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (s0 + u < a.tiles_per_seq) v += __uint_as_float(pv[u]);
        }
        v = count ? v * inv : 0.0f;
        rowv[c] = v;
        ss += (double)v * (double)v;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    if (lane == 0) dred[wave] = ss;
    __syncthreads();
    const float norm = (float)__builtin_sqrt(dred[0] + dred[1] + dred[2] + dred[3]);
    for (int c = tid; c < E3_N; c += 256) {
        float v = rowv[c];
        if (norm != 0.0f) v = v / norm;
        a.out[seq * E3_N + c] = f2h(v);
    }
    if (tid == 0) __hip_atomic_store(&a.tickets[seq], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

bool embed_gemm7_supported(const EmbedArgs& a) {
    return a.N == E3_N && a.K % 64 == 0 && a.K >= 64 && a.K <= 512;
}

hipError_t launch_embed_gemm7(const EmbedArgs& a, hipStream_t s) {
    const int64_t tiles = a.batches * a.tiles_per_seq;
    const unsigned grid = (unsigned)(tiles * 4);
    const int xcd = tiles % 8 == 0 ? 1 : 0;
    const size_t lds = (size_t)a.K * E7_BROW;
#define MANTA_EG7(NB)                                                                                    \
    case NB: {                                                                                           \
        static bool attr = false;                                                                        \
        if (!attr) {                                                                                     \
            hipError_t e = hipFuncSetAttribute((const void*)embed_gemm7_kernel<NB>,                      \
                                               hipFuncAttributeMaxDynamicSharedMemorySize,               \
                                               (int)(NB * 64 * E7_BROW));                                \
            if (e != hipSuccess) return e;                                                               \
            attr = true;                                                                                 \
        }                                                                                                \
        hipLaunchKernelGGL(embed_gemm7_kernel<NB>, dim3(grid), dim3(256), lds, s, a, xcd);               \
        return hipGetLastError();                                                                        \
    }
    switch (a.K / 64) {
        MANTA_EG7(1)
        MANTA_EG7(2)
        MANTA_EG7(3)
        MANTA_EG7(4)
        MANTA_EG7(5)
        MANTA_EG7(6)
        MANTA_EG7(7)
        MANTA_EG7(8)
    }
#undef MANTA_EG7
    return hipErrorInvalidValue;
}

// Pooled embed for large batches of short sequences (T = 64, 128 or 256):
// one workgroup of 8 waves = 256 rows (whole sequences) x all N = 384
// columns, each wave 64 rows x 192 columns (2 x 6 tiles of
// v_mfma_f32_32x32x16_f16), operands as in embed_gemm2_kernel (projection
// pre-transposed to f16 [N][K]).  A 256 x 384 tile moves 5 bytes per output
// through L2 against 9 for 256 x 128, and the tile holds whole sequences, so
// pooling, the count, the norm and the f16 store all happen in the
// workgroup: one launch after the transpose, no partials, no finalize.
constexpr int E5_WM = 256, E5_N = 384, E5_NST = 3;
constexpr int E5_AST = E5_WM * E3_KC * 2;   // 16 KB
constexpr int E5_BST = E5_N * E3_KC * 2;    // 24 KB
constexpr int E5_STAGE = E5_AST + E5_BST;

template <bool Q8B>
__global__ __launch_bounds__(512) void embed_gemm5_kernel(EmbedArgs a, const uint16_t* Bt) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ double dred[8];
    __shared__ int ired[8];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int rg = wave & 3, cg = wave >> 2;
    const int64_t row0 = (int64_t)blockIdx.x * E5_WM;  // first row of b*T
    const int K = a.K;
    // The mask of the wave's 64 rows (row 64*rg + lane of the tile; the mask
    // is [b][T], so its index is the row of b*T), loaded with the tokens so
    // the pooling after the K loop needs no global load.
    const bool live_row = !a.mask || a.mask[row0 + 64 * rg + lane] != 0;

    const uint8_t* asrc[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int r = 16 * (2 * wave + u) + (lane >> 2);
        const int idx = a.tokens[row0 + r];
        int64_t src = 0;
        if (idx >= 0 && idx < a.vocab) src = idx;
        else report_gather_error(a.err, row0 + r, idx);
        const int c = (lane & 3) ^ ((r >> 2) & 3);
        asrc[u] = (const uint8_t*)a.table + src * K * 2 + c * 16;
    }
    const uint8_t* bsrc[3];
#pragma unroll
    for (int u = 0; u < 3; u++) {
        const int n = 16 * (3 * wave + u) + (lane >> 2);
        const int c = (lane & 3) ^ ((n >> 2) & 3);
        bsrc[u] = (const uint8_t*)Bt + (int64_t)n * K * 2 + c * 16;
    }
    const uint64_t livew = __ballot(live_row);  // bit l: row 64*rg + l is unmasked
    // column scales of the six output columns this lane sums (q8 projection)
    float cscale[6];
#pragma unroll
    for (int cb = 0; cb < 6; cb++) cscale[cb] = Q8B ? a.colscale[192 * cg + 32 * cb + (lane & 31)] : 1.0f;
    const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)smem);
    auto issue = [&](int kc, int st) {
        const uint32_t sa = __builtin_amdgcn_readfirstlane(base + st * E5_STAGE + wave * 2 * 1024);
#pragma unroll
        for (int u = 0; u < 2; u++) eg_lds_load16(asrc[u] + kc * E3_KC * 2, sa + u * 1024);
        const uint32_t sb = __builtin_amdgcn_readfirstlane(base + st * E5_STAGE + E5_AST + wave * 3 * 1024);
#pragma unroll
        for (int u = 0; u < 3; u++) eg_lds_load16(bsrc[u] + kc * E3_KC * 2, sb + u * 1024);
    };
    const int nk = K / E3_KC;
#pragma unroll
    for (int st = 0; st < E5_NST - 1; st++)
        if (st < nk) issue(st, st);

    f16v acc[2][6];
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int cb = 0; cb < 6; cb++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[rb][cb][r] = 0.0f;

    const int l32 = lane & 31, hf = lane >> 5;
    int st = 0;
    for (int kc = 0; kc < nk; kc++, st = st == E5_NST - 1 ? 0 : st + 1) {
        eg_wait_barrier<5, E5_NST - 2>(nk - 1 - kc);
        if (kc + E5_NST - 1 < nk) issue(kc + E5_NST - 1, st == 0 ? E5_NST - 1 : st - 1);
        const uint8_t* As = smem + st * E5_STAGE;
        const uint8_t* Bs = As + E5_AST;
#pragma unroll
        for (int ks = 0; ks < E3_KC / 16; ks++) {
            const int c = ks * 2 + hf;
            h8 av[2];
#pragma unroll
            for (int rb = 0; rb < 2; rb++) {
                const int r = 64 * rg + 32 * rb + l32;
                av[rb] = *(const h8*)(As + r * 64 + ((c ^ ((r >> 2) & 3)) * 16));
            }
#pragma unroll
            for (int cb = 0; cb < 6; cb++) {
                const int n = 192 * cg + 32 * cb + l32;
                const h8 bv = *(const h8*)(Bs + n * 64 + ((c ^ ((n >> 2) & 3)) * 16));
#pragma unroll
                for (int rb = 0; rb < 2; rb++)
                    acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[rb], bv, acc[rb][cb], 0, 0, 0);
            }
        }
    }
    __syncthreads();  // every wave is done with the stage buffers

    // Column sums of the wave's unmasked rows (its 64 rows lie in one
    // sequence), then per sequence over its row groups in order.  Output
    // element (rb, cb, r): row 64*rg + 32*rb + 8*(r/4) + 4*(lane/32) + r%4,
    // column 192*cg + 32*cb + lane%32.
    float* part = (float*)smem;                 // [4][384]
    float* rowv = part + 4 * E5_N;              // [4][384]
    const int64_t T = a.T;
    // A wave whose 64 rows are all unmasked adds without the selects (the
    // same additions in the same order).
    const bool all_live = livew == ~0ull;
#pragma unroll
    for (int cb = 0; cb < 6; cb++) {
        float sum = 0.0f;
        if (all_live) {
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
#pragma unroll
                for (int r = 0; r < 16; r++) sum += acc[rb][cb][r];
        } else {
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    if ((livew >> (32 * rb + 8 * (r >> 2) + 4 * hf + (r & 3))) & 1u) sum += acc[rb][cb][r];
        }
        sum += __shfl_xor(sum, 32);
        const int n = 192 * cg + 32 * cb + l32;
        if (hf == 0) part[rg * E5_N + n] = Q8B ? sum * cscale[cb] : sum;
    }
    if (cg == 0 && lane == 0) ired[rg] = __popcll(livew);  // unmasked rows of row group rg
    __syncthreads();
    // 128 threads per sequence (at most 4 sequences of the tile)
    const int S = (int)(E5_WM / T);
    const int sl = tid >> 7, j = tid & 127;
    const int gps = (int)(T / 64);  // row groups per sequence
    const int64_t seq = row0 / T + sl;
    int count = 0;
    if (sl < S)
        for (int g2 = 0; g2 < gps; g2++) count += ired[sl * gps + g2];
    const float inv = count ? 1.0f / (float)count : 0.0f;
    double ss = 0.0;
    if (sl < S) {
        for (int c = j; c < E5_N; c += 128) {
            float v = 0.0f;
            for (int g2 = 0; g2 < gps; g2++) v += part[(sl * gps + g2) * E5_N + c];
            v = count ? v * inv : 0.0f;
            rowv[sl * E5_N + c] = v;
            ss += (double)v * (double)v;
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    if (lane == 0) dred[wave] = ss;
    __syncthreads();
    if (sl < S) {
        const float norm = (float)__builtin_sqrt(dred[2 * sl] + dred[2 * sl + 1]);
        for (int c = j; c < E5_N; c += 128) {
            float v = rowv[sl * E5_N + c];
            if (norm != 0.0f) v = v / norm;
            a.out[seq * E5_N + c] = f2h(v);
        }
    }
}

bool embed_gemm5_supported(const EmbedArgs& a) {
    return a.N == E5_N && a.K % E3_KC == 0 && a.K > 0 && (a.T == 64 || a.T == 128 || a.T == 256) &&
           (a.batches * a.T) % E5_WM == 0;
}

hipError_t launch_embed_gemm5(const EmbedArgs& a, bool q8b, const uint16_t* Bt, hipStream_t s) {
    const size_t lds = (size_t)E5_NST * E5_STAGE;
    const unsigned grid = (unsigned)(a.batches * a.T / E5_WM);
#define MANTA_EG5(Q)                                                                                   \
    if (q8b == Q) {                                                                                    \
        static bool attr = false;                                                                      \
        if (!attr) {                                                                                   \
            hipError_t e = hipFuncSetAttribute((const void*)embed_gemm5_kernel<Q>,                     \
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds); \
            if (e != hipSuccess) return e;                                                             \
            attr = true;                                                                               \
        }                                                                                              \
        hipLaunchKernelGGL((embed_gemm5_kernel<Q>), dim3(grid), dim3(512), lds, s, a, Bt);              \
        return hipGetLastError();                                                                      \
    }
    MANTA_EG5(true)
    MANTA_EG5(false)
#undef MANTA_EG5
    return hipErrorInvalidValue;
}

bool embed_gemm3_supported(const EmbedArgs& a, bool q8b) {
    return !q8b && a.N == E3_N && a.K % E3_KC == 0 && a.K > 0;
}

hipError_t launch_embed_gemm3(const EmbedArgs& a, bool gather, bool pool, hipStream_t s) {
    const int64_t tiles = pool ? a.batches * a.tiles_per_seq : (a.M + E3_WM - 1) / E3_WM;
    const size_t lds = (size_t)E3_NST * E3_STAGE;
#define MANTA_EG3(G, P)                                                                                \
    if (gather == G && pool == P) {                                                                    \
        static bool attr = false;                                                                      \
        if (!attr) {                                                                                   \
            hipError_t e = hipFuncSetAttribute((const void*)embed_gemm3_kernel<G, P>,                  \
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds); \
            if (e != hipSuccess) return e;                                                             \
            attr = true;                                                                               \
        }                                                                                              \
        hipLaunchKernelGGL((embed_gemm3_kernel<G, P>), dim3((unsigned)tiles), dim3(256), lds, s, a);   \
        return hipGetLastError();                                                                      \
    }
    MANTA_EG3(true, true)
    MANTA_EG3(false, false)
    MANTA_EG3(true, false)
#undef MANTA_EG3
    return hipErrorInvalidValue;
}

bool embed_gemm2_supported(const EmbedArgs& a) { return a.K % EG_KC == 0 && a.K > 0 && a.N % EG_WN == 0 && a.N > 0; }

size_t embed_gemm2_lds() { return (size_t)EG_NST * EG_STAGE; }

hipError_t launch_embed_transpose_b(const EmbedArgs& a, bool q8b, uint16_t* Bt, hipStream_t s) {
    hipLaunchKernelGGL(embed_transpose_b_kernel, dim3((unsigned)((a.N + 31) / 32), (unsigned)((a.K + 31) / 32)),
                       dim3(256), 0, s, a.B, q8b ? 1 : 0, a.K, a.N, Bt);
    return hipGetLastError();
}

hipError_t launch_embed_gemm2(const EmbedArgs& a, bool gather, bool q8b, bool pool, const uint16_t* Bt,
                              hipStream_t s) {
    const int64_t tiles = pool ? a.batches * a.tiles_per_seq : (a.M + EG_WM - 1) / EG_WM;
    dim3 grid((unsigned)((tiles + 3) / 4), (unsigned)(a.N / EG_WN));
    const size_t lds = embed_gemm2_lds();
#define MANTA_EG2(G, Q, P)                                                                          \
    if (gather == G && q8b == Q && pool == P) {                                                     \
        hipLaunchKernelGGL((embed_gemm2_kernel<G, Q, P>), grid, dim3(256), lds, s, a, Bt);                \
        return hipGetLastError();                                                                   \
    }
    MANTA_EG2(true, false, true)
    MANTA_EG2(true, true, true)
    MANTA_EG2(false, false, false)
    MANTA_EG2(false, true, false)
    MANTA_EG2(true, false, false)
    MANTA_EG2(true, true, false)
#undef MANTA_EG2
    return hipErrorInvalidValue;
}

hipError_t launch_embed_gemm(const EmbedArgs& a, bool gather, bool q8b, bool pool, hipStream_t s) {
    const int64_t rows_tiles = pool ? a.batches * a.tiles_per_seq : (a.M + EM - 1) / EM;
    dim3 grid((unsigned)rows_tiles, (unsigned)((a.N + EN - 1) / EN));
#define MANTA_EG(G, Q, P) \
    if (gather == G && q8b == Q && pool == P) { \
        hipLaunchKernelGGL((embed_gemm_kernel<G, Q, P>), grid, dim3(256), 0, s, a); \
        return hipGetLastError(); \
    }
    MANTA_EG(true, false, true)
    MANTA_EG(true, true, true)
    MANTA_EG(false, false, false)
    MANTA_EG(false, true, false)
    MANTA_EG(true, false, false)
    MANTA_EG(true, true, false)
#undef MANTA_EG
    return hipErrorInvalidValue;
}

hipError_t launch_embed_finalize(const float* P, int tiles, const int32_t* mask, int64_t B, int64_t T,
                                 int N, uint16_t* out, hipStream_t s) {
    hipLaunchKernelGGL(embed_finalize_kernel, dim3((unsigned)B), dim3(256), 0, s, P, tiles, mask, T, N, out);
    return hipGetLastError();
}

hipError_t launch_gather_rows_f16(const uint16_t* table, int64_t vocab, int64_t d, const int32_t* idx,
                                  int64_t nidx, uint16_t* out, unsigned long long* err, hipStream_t s) {
    hipLaunchKernelGGL(gather_rows_f16_kernel, dim3((unsigned)nidx), dim3(128), 0, s, table, vocab, d, idx,
                       nidx, out, err);
    return hipGetLastError();
}

hipError_t launch_mean_pool_masked(const float* x, const int32_t* mask, int64_t B, int64_t T, int64_t C,
                                   float* out, hipStream_t s) {
    const int64_t total = B * C;
    hipLaunchKernelGGL(mean_pool_masked_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, x,
                       mask, B, T, C, out);
    return hipGetLastError();
}

// normalizeRows with coalesced traffic: a workgroup stages rb rows in LDS
// (row pitch cols + 1 words, so the summing threads hit distinct banks), one
// thread per row sums the squares sequentially in f64 in column order -- the
// same operations in the same order as normalize_rows_kernel -- and all
// threads divide and write back.
__global__ __launch_bounds__(256) void normalize_rows_lds_kernel(float* __restrict__ x, int64_t rows, int cols,
                                                                 int rb) {
    extern __shared__ float L[];  // [rb][cols + 1], then rb norms
    const int pitch = cols + 1;
    float* norms = L + (int64_t)rb * pitch;
    const int64_t r0 = (int64_t)blockIdx.x * rb;
    const int nr = (int)(rows - r0 < rb ? rows - r0 : rb);
    const int n = nr * cols;
    for (int i = threadIdx.x; i < n; i += 256) {
        const int r = i / cols, c = i - r * cols;
        L[r * pitch + c] = x[(r0 + r) * cols + c];
    }
    __syncthreads();
    if ((int)threadIdx.x < nr) {
        const float* p = L + threadIdx.x * pitch;
        double s = 0.0;
        for (int c = 0; c < cols; c++) {
            const double v = (double)p[c];
            s = __dadd_rn(s, __dmul_rn(v, v));
        }
        norms[threadIdx.x] = (float)__builtin_sqrt(s);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += 256) {
        const int r = i / cols, c = i - r * cols;
        const float norm = norms[r];
        if (norm != 0.0f) x[(r0 + r) * cols + c] = fdiv_rn(L[r * pitch + c], norm);
    }
}

hipError_t launch_normalize_rows(float* x, int64_t rows, int64_t cols, hipStream_t s) {
    // rows per workgroup: as many as 64 KB of LDS holds, at most 32
    const int64_t rb = cols + 1 <= 16384 ? std::min<int64_t>(32, 16384 / (cols + 1)) : 0;
    if (rb >= 1 && cols <= 0x7FFFFFFF / 32) {
        const size_t lds = ((size_t)rb * (size_t)(cols + 1) + (size_t)rb) * sizeof(float);
        hipLaunchKernelGGL(normalize_rows_lds_kernel, dim3((unsigned)((rows + rb - 1) / rb)), dim3(256), lds, s, x,
                           rows, (int)cols, (int)rb);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(normalize_rows_kernel, dim3((unsigned)((rows + 63) / 64)), dim3(64), 0, s, x, rows,
                       cols);
    return hipGetLastError();
}

}  // namespace manta
