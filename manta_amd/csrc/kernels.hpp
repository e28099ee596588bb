// kernels.hpp -- host-side launchers of the gfx950 kernels (internal to
// libmanta_rocm.so; the public surface is include/manta_rocm.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace manta {

// Device score ops.  OP_DOT / OP_COSINE / OP_L2 name the reference's
// dotRows / cosineRows / l2DistanceRows where a kernel computes those
// (kernels_ref.hip); in the quantized-query scans they name the scan's own
// score: q8 OP_DOT with E8 query codes (BASELINE's q8 dot formula), every
// other q8 op and every q4 op with E16 codes.  OP_DOT16 is the q8 dot with
// E16 codes (qd), a scan score only.
enum { OP_DOT = 0, OP_COSINE = 1, OP_L2 = 2, OP_DOT16 = 3 };

struct QConst;

constexpr int kMaxQueryDim = 1024;  // longest query / row the device path takes
constexpr int kMaxCapKeys = 4096;   // largest LDS key reservoir (32 KB)
constexpr int kWaveListMaxK = 64;   // largest k kept in per-wave register lists

// Arguments of the streaming scan kernels (one query per blockIdx.y).
struct ScanArgs {
    const int8_t* codes;      // q8: [sets][n][pitch] int8; q4: [sets][n][pitch] packed bytes
    const void* scales;       // q8: f32 [sets][n]; q4: f16 [sets][n][nb]
    const float* dnorm;       // [sets][n]
    const float* dd;          // [sets][n]
    int64_t n;
    int pitch;                // bytes per row
    int nb;                   // q4 blocks per row
    int d;                    // query length
    int64_t set_stride;       // rows between consecutive queries' sets (0: shared)
    const uint16_t* queries;  // f16 [nq][d]
    int rounds;               // rounds of 256 rows per workgroup
    float* out_scores;        // score-matrix mode, else nullptr
    uint64_t* partial;        // top-k mode: [nq][gridDim.x][k]
    uint32_t* tickets;        // [nq], zero between calls
    int32_t* out_ids;         // [nq][k]
    float* out_topk_scores;   // [nq][k] or nullptr
    int k;
    int cap;                  // reservoir capacity (power of two, >= k + 256)
    int lds_keys;             // keys the dynamic LDS holds (>= cap; merge fast path)
    int mid_compact;          // 0: cap >= k + rounds*256, no compaction between rounds
    int smallest;
    int wave_lists;           // 1: k <= 64 top lists held in registers (coalesced q8 kernel only)
};

// Query codes for the batched paths (one workgroup per query).  With tau
// and bcnt given it also resets the threshold passes' per-query state
// (tau[q] = 0, bcnt[q] = 0) before the first pass, saving a launch.
hipError_t launch_query_encode(const uint16_t* q, int nq, int d, int pitch, int e16, int8_t* c8,
                               int8_t* hi, int8_t* lo, QConst* qc, uint64_t* tau, int* bcnt, hipStream_t s);

// Error bounds of the int8 shadow of a q4 matrix: maxima over its rows of
// E_r = |x_r - t_r e_r| and F_r = t_r |e_r| (x_r the dequantized q4 row, e_r
// its int8 codes, t_r their scale), divided by |x_r| for cosine, and of
// |x_r|; f32 bit patterns (non-negative, so integer max is float max),
// rounded up.
struct ShadowInfo {
    unsigned int me_cos, mf_cos;
    unsigned int me_dot, mf_dot;
    unsigned int maxn;
    unsigned int pad[3];
};
// Build the shadow of n q4 rows of length d (d <= 384): int8 codes
// [n][spitch] (zero padded), per-row scales t_r (dot) and t_r / dnorm_r
// (cosine), and the bounds (info must hold zeros; see launch_shadow_info_clear).
hipError_t launch_shadow_info_clear(ShadowInfo* info, hipStream_t s);
hipError_t launch_q4_shadow_build(const uint8_t* packed, const uint16_t* scales, const float* dnorm, int64_t n,
                                  int d, int spitch, int8_t* codes, float* sc_dot, float* sc_cos,
                                  ShadowInfo* info, hipStream_t s);
// Queries for the shadow scan: full-range int8 codes c8 [nq][spitch] with
// qa = maxabs/127, E16 digit planes in the q4 order hi/lo [nq][d], E16
// constants qc, and per query the margin m and factor f of shadow_bound for
// op (OP_COSINE or OP_DOT): qb[2q] = m, qb[2q+1] = f.
// tau / bcnt as for launch_query_encode.
hipError_t launch_query_encode_shadow(const uint16_t* q, int nq, int d, int spitch, int op, const ShadowInfo* info,
                                      int8_t* c8, int8_t* hi, int8_t* lo, QConst* qc, float* qb, uint64_t* tau,
                                      int* bcnt, hipStream_t s);
hipError_t launch_q8_scan(int op, const ScanArgs& a, dim3 grid, size_t lds, hipStream_t s);
// Pitches served by the coalesced q8 kernel (the others use the row-per-lane one).
bool q8_scan_coalesced(int pitch);
hipError_t launch_q4_scan(int op, const ScanArgs& a, dim3 grid, size_t lds, hipStream_t s);
hipError_t launch_q8_rescore(const int8_t* codes, int pitch, int64_t set_stride, int64_t n, int d,
                             const uint16_t* queries, const int32_t* ids, int k, int nq, int e16,
                             int64_t* out, hipStream_t s);

// ---- reference scores (kernels_ref.hip)
//
// A quantized-query scan returns the best kp >= k rows of each query by its
// own score; ref_finish rescores them with the reference's arithmetic
// (ref_common.hpp), keeps the best k and proves from the scan score of the
// kp-th row and the error bounds that no other row can reach them.  A query
// where the proof fails (ties or near-ties across the kp-th row, or
// non-finite inputs) is marked for ref_scan, which rescans every row with
// the reference arithmetic, starting from the k-th best reference score the
// finish found.
struct RefArgs {
    int fmt;                    // 8: q8 rows, 4: q4 blocks
    const void* codes;          // q8 [sets][n][pitch] int8; q4 [sets][n][d/2] bytes
    const void* scales;         // q8 f32 [sets][n]; q4 f16 [sets][n][d/32]
    const double* sqd;          // [sets][n] sqrt of each row's f64 square-sum
    int64_t n;
    int pitch;                  // bytes per row
    int d;
    int64_t set_stride;         // rows between consecutive queries' sets (0: shared)
    const uint16_t* queries;    // f16 [nq][d]
    int nq;
    int op;                     // OP_DOT, OP_COSINE or OP_L2 (reference semantics)
    int smallest;
    int k;
    int kp;                     // scan rows per query (k <= kp <= n)
    const int32_t* cand_ids;    // [nq][kp] the scan's best rows, in any order but the worst last
    const float* cand_scores;   // [nq][kp] their scan scores (position kp-1: the worst)
    float e_qd;                 // relative error bound of the scan's q^.d' term
    float maxdn;                // max over rows of |d'|, as stored
    float maxdd;                // max over rows of |d'|^2, as stored
    int32_t* out_ids;           // [nq][k]
    float* out_scores;          // [nq][k] or nullptr
    int* redo;                  // [nq] 1: the query goes to ref_scan
    uint64_t* redo_tau;         // [nq] threshold key ref_scan starts from (0: none)
};
// keys [nq][kp]: the reference key of each candidate (ref_rescore), then
// the finish over them.
hipError_t launch_ref_rescore(const RefArgs& a, uint64_t* keys, hipStream_t s);
hipError_t launch_ref_finish(const RefArgs& a, const uint64_t* keys, hipStream_t s);
// Reference scores of every row (score matrix: a.out_scores, grid
// (parts, nq)) or top-k with the streaming reservoir and last-workgroup merge
// (ScanArgs as for the streaming scans; grid (parts, R), each blockIdx.y
// taking every R-th query).  redo / redo_tau (may be null: every query, no
// bound).
hipError_t launch_ref_scan(int fmt, int op, const ScanArgs& a, int nq, const double* sqd, const int* redo,
                           const uint64_t* redo_tau, dim3 grid, size_t lds, hipStream_t s);

// Arguments of the multi-query scan kernel (kernels_mq.hip): nq queries
// against one shared candidate matrix, over rows [row_begin, row_end).
struct MqArgs {
    const int8_t* codes;        // q8 [n][pitch]
    const float* scales;        // [n]
    const float* dnorm;         // [n]
    const float* dd;            // [n]
    int64_t n;
    int pitch;                  // bytes per row, multiple of 32
    int64_t row_begin;          // rows of this pass
    int64_t row_end;
    int64_t rows_per_wg;        // rows per blockIdx.x (multiple of the chunk)
    int nq;
    const int8_t* qc8;          // E8 codes [nq][pitch]
    const int8_t* qhi;          // E16 digits [nq][pitch]
    const int8_t* qlo;
    const QConst* qconst;       // [nq]
    const uint64_t* tau;        // [nq] threshold keys of this pass (0: none)
    uint64_t* regions;          // [R][nq][rc] appended keys (nq*R*rc < 2^31)
    int* counts;                // [R][nq] keys per region
    int R;                      // gridDim.x
    int rc;                     // region capacity (>= k + 2 * chunk rows + 1)
    int k;
    float* out_scores;          // score-matrix mode [nq][n], else nullptr
    int smallest;
    // int8 shadow of a q4 matrix (mq8 kernel, shadow mode): codes / scales
    // above are the shadow's, these the q4 matrix's for exact rescoring
    const float* qbound;        // [nq][2] margin m and factor f (shadow_bound)
    const uint8_t* q4codes;     // [n][d/2]
    const uint16_t* q4scales;   // [n][d/32]
    int d;
    int op;                     // OP_COSINE or OP_DOT
    // mq8 kernel, first top-k pass (no threshold yet): every (query, row)
    // pair goes to its region at the row's offset in the workgroup's range,
    // without tests or atomics (rows_per_wg <= rc)
    int keep_all;
};

// Arguments of the per-query merge after a pass.
struct MqSelectArgs {
    const uint64_t* regions;    // [R][nq][rc]
    const int* counts;          // [R][nq]
    int R;
    int rc;
    uint64_t* best;             // [nq][k] best keys so far (sorted), updated
    int* bcnt;                  // [nq] valid keys in best
    uint64_t* tau;              // [nq] next pass's threshold key (0: none)
    int k;
    int nq;
    int32_t* out_ids;           // final pass: [nq][k] ids (else nullptr)
    float* out_scores;          // final pass: [nq][k] scores or nullptr
    int smallest;
    int pairs;                  // region entries: 0 keys; 1 q8 dot pairs (bits of p = scale*acc) << 32 | row,
                                // the key's score p*qmax/127; 2 shadow pairs, the key the exact q4 score
    int uniform;                // > 0: every region but the last holds exactly this many entries
                                // (a pass that keeps every pair), so entry g is in region g / uniform
    const QConst* qconst;       // [nq] (pairs 1: E8 qmax; pairs 2: E16 constants)
    // pairs 2: the q4 matrix and the E16 digit planes in the q4 order [nq][d]
    const uint8_t* q4codes;
    const uint16_t* q4scales;
    const float* dnorm;
    const float* dd;
    const int8_t* qhi;
    const int8_t* qlo;
    const float* qbound;        // [nq][2] the shadow margin m and factor f
    int d;
    int op;
    int unsorted;               // final pass: ids / scores in any order, the k-th best (the worst kept) last
};

// Launch shape of the scan kernel for an op, K steps (pitch / 32) and query count.
struct MqShape {
    int kind = 0;        // 0: mq_scan / mq_q4 (256 threads); 1: mq8_scan (512 threads, q8 dot or q4 shadow)
    int ws = 1;          // kind 1: wave groups splitting a chunk's rows (queries per workgroup 512 / ws)
    int shadow = 0;      // kind 1: q4 shadow mode
    int ks = 0;
    int na = 0;          // A blocks per wave
    int wq = 0;          // waves splitting the queries (1 or 4)
    int qg = 0;          // queries per workgroup
    int chunk = 0;       // candidate rows per LDS chunk
    int tile = 0;        // LDS bytes of one chunk tile
    int tile_bytes = 0;  // LDS bytes of all chunk tiles and their row constants
    int threads = 256;   // workgroup size
};

MqShape mq_shape(int op, int ks, int64_t nq);
bool mq_supported_ks(int ks);
hipError_t launch_mq_scan(int op, const MqShape& sh, const MqArgs& a, dim3 grid, size_t lds, hipStream_t s);
// q4 blocks (kernels_mq4.hip): codes = packed nibbles [n][nb*16], scales =
// f16 [n][nb] (passed through MqArgs.scales), qhi/qlo = E16 planes in the q4
// nibble order [nq][nb*32]; MqShape.ks holds nb.
MqShape mq4_shape(int op, int nb, int64_t nq);
bool mq4_supported_nb(int nb);
hipError_t launch_mq4_scan(int op, const MqShape& sh, const MqArgs& a, dim3 grid, size_t lds, hipStream_t s);
// q8 dot with many queries (kernels_mq8.hip): 512-thread workgroups of 512
// (ws 1) or 256 (ws 2) queries on 16x16x64 i8 MFMAs, top-k mode only; pitch
// 128, 256 or 384.  Shadow mode scans the int8 shadow of a q4 matrix.
bool mq8_supported(int pitch);
MqShape mq8_shape(int pitch, int ws, bool shadow);
hipError_t launch_mq8_scan(const MqShape& sh, const MqArgs& a, dim3 grid, size_t lds, hipStream_t s);
int mq_select_threads(int64_t expect_keys);
size_t mq_select_lds(int threads, int R);
hipError_t launch_mq_select(const MqSelectArgs& a, int threads, hipStream_t s);

// Candidate pack after top-k (kernels_topk.hip).
struct PackArgs {
    const int32_t* top;         // [nq][k] row indices
    int64_t nq, k, n;
    int sets;                   // 1 (shared rows) or nq (set q per query)
    const uint8_t* codes;       // [sets][n][pitch]
    int64_t pitch;              // bytes between rows
    int row_bytes;              // bytes copied per row
    const uint8_t* scales;      // [sets][n][scale_bytes]
    int scale_bytes;
    const int64_t* ids;         // [sets][n] or nullptr
    int64_t* ids_out;           // [nq][k] or nullptr
    uint8_t* rows_out;          // [nq][k][row_bytes]
    uint8_t* scales_out;        // [nq][k][scale_bytes]
    unsigned long long* err;    // first out-of-range index
};
hipError_t launch_pack_candidates(const PackArgs& a, hipStream_t s);

// Arguments of the embed GEMM kernels (kernels_embed.hip).
struct EmbedArgs {
    const int32_t* tokens;      // [batches*T] (pooled) or [M] (gathered matmul)
    const int32_t* mask;        // [batches*T] or nullptr (all positions valid)
    const void* table;          // f16 [vocab][K]
    int64_t vocab;
    const void* A;              // plain f16 lhs [M][K]
    int64_t M;                  // rows of a plain / gathered matmul
    int64_t T;                  // positions per sequence (pooled)
    int64_t batches;            // sequences (pooled)
    int tiles_per_seq;          // ceil(T / 64)
    int K;
    int N;
    const void* B;              // f16 [K][N] or int8 [K][N]
    const float* colscale;      // [N] for int8 B
    float* Y;                   // f32 [M][N] (matmul)
    float* P;                   // f32 [batches][tiles_per_seq][N] (pooled partial sums)
    unsigned long long* err;    // first out-of-range gather index
    unsigned int* tickets;      // [batches] zero between calls (single-pass pooled kernel)
    uint16_t* out;              // f16 [batches][N] embeddings (single-pass pooled kernel)
    uint16_t* Y16;              // plain matmul of embed_gemm2: f16 [M][N] output instead of Y (or nullptr)
    int gelu;                   // with Y16: geluTensor (tanh in f32) applied to each value before the f16 rounding
};

hipError_t launch_embed_gemm(const EmbedArgs& a, bool gather, bool q8b, bool pool, hipStream_t s);
// Pipelined GEMM for K % 32 == 0 and N % 128 == 0: launch_embed_transpose_b
// writes the projection as Bt (f16 [N][K], N*K*2 bytes, int8 codes widened
// exactly), then launch_embed_gemm2 runs 256-row x 128-column workgroup tiles
// over it; same outputs as launch_embed_gemm.
bool embed_gemm2_supported(const EmbedArgs& a);
hipError_t launch_embed_transpose_b(const EmbedArgs& a, bool q8b, uint16_t* Bt, hipStream_t s);
hipError_t launch_embed_gemm2(const EmbedArgs& a, bool gather, bool q8b, bool pool, const uint16_t* Bt,
                              hipStream_t s);
// Single-pass GEMM for an f16 projection with N == 384 and K % 32 == 0: the
// projection is read as stored ([K][N]) through LDS transpose reads, one
// workgroup per 32-row tile.  Pooled mode (tiles_per_seq = ceil(T / 32))
// also finishes the embeddings: partial sums go to P, and the last tile of
// each sequence writes out[seq] (tickets must hold zeros; they are reset).
bool embed_gemm3_supported(const EmbedArgs& a, bool q8b);
hipError_t launch_embed_gemm3(const EmbedArgs& a, bool gather, bool pool, hipStream_t s);
// The pooled embed of embed_gemm3 with 128-row x 96-column tiles
// (tiles_per_seq = ceil(T / 128); same requirements, P and tickets).
hipError_t launch_embed_gemm4(const EmbedArgs& a, hipStream_t s);
// The same pooled embed with every operand loaded in one round (the
// projection slice to LDS, the gathered rows to registers): N == 384,
// K % 64 == 0, K <= 512; tiles_per_seq = ceil(T / 128); P holds
// [batches*tiles_per_seq][N] partial sums followed by [batches*tiles_per_seq]
// unmasked counts.
bool embed_gemm7_supported(const EmbedArgs& a);
hipError_t launch_embed_gemm7(const EmbedArgs& a, hipStream_t s);
// Pooled embed with the projection pre-transposed (launch_embed_transpose_b)
// for N == 384, K % 32 == 0, T in {64, 128, 256} and batches*T a multiple of
// 256: 256-row workgroups of whole sequences finish their embeddings in one
// launch (no P, no tickets).
bool embed_gemm5_supported(const EmbedArgs& a);
hipError_t launch_embed_gemm5(const EmbedArgs& a, bool q8b, const uint16_t* Bt, hipStream_t s);
hipError_t launch_embed_finalize(const float* P, int tiles, const int32_t* mask, int64_t B, int64_t T,
                                 int N, uint16_t* out, hipStream_t s);
hipError_t launch_gather_rows_f16(const uint16_t* table, int64_t vocab, int64_t d, const int32_t* idx,
                                  int64_t nidx, uint16_t* out, unsigned long long* err, hipStream_t s);
hipError_t launch_mean_pool_masked(const float* x, const int32_t* mask, int64_t B, int64_t T, int64_t C,
                                   float* out, hipStream_t s);
hipError_t launch_normalize_rows(float* x, int64_t rows, int64_t cols, hipStream_t s);

// encoder steps (kernels_encoder.hip)
// x16 / y16 / C16 (optional): the same values rounded to f16 as well, the
// left operand of the f16 weight GEMMs
hipError_t launch_enc_gather_q8(const int32_t* tok, int64_t rows, const int8_t* codes, const float* scales,
                                int64_t vocab, int d, float* x, unsigned long long* err, hipStream_t s,
                                uint16_t* x16 = nullptr);
hipError_t launch_enc_gemm(int bmode, const float* A, int64_t sA, const void* B, const float* bscale, int64_t sB,
                           float* C, int64_t sC, int M, int N, int K, int batches, hipStream_t s, bool gelu = false,
                           uint16_t* C16 = nullptr);
hipError_t launch_enc_softmax_rows(float* x, int64_t rows, int cols, hipStream_t s);
hipError_t launch_enc_add_layernorm(const float* a, const float* b, float* y, int64_t rows, int cols,
                                    hipStream_t s, uint16_t* y16 = nullptr);
hipError_t launch_enc_to_f16(const float* x, int64_t n, uint16_t* out, hipStream_t s);
hipError_t launch_enc_gelu(float* x, int64_t n, hipStream_t s);

hipError_t launch_topk_rows_partial(const float* scores, int64_t rows, int64_t cols, int64_t seg,
                                    int parts, int k, int cap, int smallest, uint64_t* partial,
                                    hipStream_t s);
hipError_t launch_topk_merge(const uint64_t* partial, int64_t rows, int64_t per_row, int k, int cap,
                             int smallest, int32_t* ids, float* values, hipStream_t s);

// dotRetrievalVectors score matrix (kernels_dense.hip)
hipError_t launch_dense_dot(const void* rows, int f16, int64_t n, int64_t pitch, int len, const float* queries,
                            int64_t qpitch, int nq, float* out, hipStream_t s);

// artifact executor steps (kernels_exec.hip)
hipError_t launch_gather_elems(const void* table, int elem_bytes, int64_t rows, int64_t cols, int64_t bstride,
                               const int32_t* idx, int64_t B, int64_t K, void* out, unsigned long long* err,
                               hipStream_t s);
hipError_t launch_widen_f16(const uint16_t* in, float* out, int64_t n, hipStream_t s);
hipError_t launch_mean_pool(const float* x, int64_t B, int64_t T, int64_t C, float* out, hipStream_t s);
// transposeTensor of [B][R][C] elements of elem_bytes -> [B][C][R]
hipError_t launch_transpose(const void* in, int elem_bytes, int64_t B, int64_t R, int64_t C, void* out,
                            hipStream_t s);
// binaryTensorOp: op 0 add, 1 sub, 2 mul, 3 div (f32, elementwise)
hipError_t launch_binary_f32(int op, const float* a, const float* b, float* out, int64_t n, hipStream_t s);
// q8 codes to f32 values: code * scale, the scale per row (per_col 0, rows
// of `cols` codes) or per column (per_col 1)
hipError_t launch_dequant_q8(const int8_t* codes, const float* scales, int64_t rows, int64_t cols, int per_col,
                             float* out, hipStream_t s);

}  // namespace manta
