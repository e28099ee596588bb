/*
 * manta_rocm.h -- C ABI of libmanta_rocm.so, the MI355X (gfx950) backend for
 * Manta's retrieval hot path: packed q8/q4 candidate scoring (dot, cosine,
 * l2_distance with dequantization fused into the kernel), top-k selection, and
 * the embed pipeline (gather -> @matmul -> masked mean_pool -> normalize).
 *
 * The reference (odvcencio/manta, Go) reaches its CUDA device through a cgo C
 * preamble in runtime/backends/cuda/native_linux.go.  This header is the
 * equivalent surface for a `runtime/backends/rocm` cgo package; each entry
 * point names the reference function it takes over.
 *
 * Conventions (same as the reference shim, native_linux.go:30-75,620-624):
 *   - every fallible call returns MANTA_ROCM_OK (0) or an error code and, on
 *     error, stores a malloc'd message in *err (if err != NULL) that the
 *     caller releases with manta_rocm_free_error;
 *   - MANTA_ROCM_UNSUPPORTED marks a shape the device path does not take;
 *     the Go side then runs the host reference with
 *     execution_mode=host_fallback, as cuda.go:248-257 does;
 *   - a runtime is bound to one device and owns one HIP stream; calls are
 *     asynchronous on that stream unless they return host data; one runtime
 *     must not be used from two threads at once (the reference's
 *     deviceRuntime has the same rule, cuda.go:69-71);
 *   - "_dev" pointers are device addresses (from manta_rocm_malloc or any
 *     HIP allocation on the runtime's device); other pointers are host.
 *
 * Packed formats (this library's contract; the reference has only
 * f32-backed fake-quantized q4/q8, runtime/backend/tensor.go:49-71):
 *   q8 rows   [n, d] int8 codes + f32 scale per row.
 *   q4 blocks [n, d/2] bytes, two's-complement nibbles, low nibble first,
 *             blocks of 32 along d, f16 scale per block ([n, d/32]).
 */
#ifndef MANTA_ROCM_H
#define MANTA_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MANTA_ROCM_ABI_VERSION 2

enum {
    MANTA_ROCM_OK = 0,
    MANTA_ROCM_ERROR = 1,
    MANTA_ROCM_UNSUPPORTED = 2,
};

/* Score builtins: the kernel body op names dot / cosine / l2_distance
 * (compiler/compiler.go:803-842, classified at native_linux.go:1734-1750).
 *
 * By default every score is the reference's own arithmetic on the values the
 * packed candidates stand for, bit for bit: dotRows (f32 sum in column
 * order), cosineRows (f64 dot and norms, narrowed), l2DistanceRows (f32
 * difference, f64 square-sum, sqrt, narrowed) of tensor_ops.go:1366-1490,
 * with a q8 element valued code*scale in f32 and a q4 element code*f16scale
 * (the f32 values a fake-quantized reference tensor holds,
 * runtime/embedding_trainer.go:3753-3762) and the f16 query widened to f32.
 * Top-k ids are topKTensor's (value desc, index asc).
 *
 * OR-ing MANTA_ROCM_QUANTIZED_QUERY into the op selects this library's
 * quantized-query scores instead: q8 dot is BASELINE's formula
 * (query codes round(q*127/max(1, maxabs q)), int32 accumulation,
 * score = scale*acc*qmax/127 in f32); the other ops use 16-bit query codes
 * (round(q*32639/maxabs q)) with exact integer accumulation.  Within a
 * stated bound of the reference scores, not equal to them. */
enum {
    MANTA_ROCM_DOT = 0,
    MANTA_ROCM_COSINE = 1,
    MANTA_ROCM_L2_DISTANCE = 2,
    MANTA_ROCM_QUANTIZED_QUERY = 0x100,
};

/* Selection order.  LARGEST is topKTensor's order (value desc, index asc;
 * runtime/backend/tensor_ops.go:1539-1551).  SMALLEST (value asc, index asc)
 * is the smallest-k extension an l2 rerank needs. */
enum {
    MANTA_ROCM_LARGEST = 0,
    MANTA_ROCM_SMALLEST = 1,
};

enum {
    MANTA_ROCM_Q8_ROWS = 8,
    MANTA_ROCM_Q4_BLOCKS = 4,
};

/* Dense retrieval vectors (manta_rocm_dense_*). */
enum {
    MANTA_ROCM_DENSE_F32 = 32,
    MANTA_ROCM_DENSE_F16 = 16, /* IEEE binary16 bits, widened exactly */
};

/* Projection kinds for the embed pipeline. */
enum {
    MANTA_ROCM_PROJ_F16 = 0,    /* f16 [d, e] */
    MANTA_ROCM_PROJ_Q8_COL = 1, /* int8 [d, e] + f32 scale per output column */
    /* the two above prepared once by manta_rocm_prepare_projection: f16
     * [e, d], the matrix cores' operand layout (int8 codes widened exactly,
     * the column scales still applied after accumulation) */
    MANTA_ROCM_PROJ_F16_T = 2,
    MANTA_ROCM_PROJ_Q8_COL_T = 3, /* + f32 scale per output column */
};

typedef struct MantaRocm MantaRocm;
typedef struct MantaRocmCandidates MantaRocmCandidates;

typedef struct {
    uint64_t kernel_launches;
    uint64_t bytes_uploaded;
    uint64_t bytes_downloaded;
    uint64_t workspace_bytes;
    uint64_t candidate_bytes;
} MantaRocmStats;

int manta_rocm_abi_version(void);

/* ---- runtime ---------------------------------------------------------- */

/* Number of visible HIP devices (0 when none). */
int manta_rocm_device_count(int* out, char** err);

/* Replaces mantaCudaRuntimeCreate (native_linux.go:108-169): binds device
 * `device`, creates the runtime's stream. */
int manta_rocm_create(int device, MantaRocm** out, char** err);

/* Replaces mantaCudaRuntimeDestroy (native_linux.go:171-189).  Candidate
 * sets still bound on the runtime lose their device memory with it; their
 * handles stay valid only for manta_rocm_unbind, which then frees the handle
 * alone. */
void manta_rocm_destroy(MantaRocm* rt);

/* Replaces mantaCudaFreeCString (native_linux.go:620-624). */
void manta_rocm_free_error(char* msg);

/* Use an external HIP stream (hipStream_t) for all later work, or NULL for
 * the runtime's own stream.  No reference counterpart (the CUDA shim always
 * uses the legacy stream, native_linux.go:391). */
int manta_rocm_set_stream(MantaRocm* rt, void* hip_stream, char** err);

/* Replaces mantaCudaSynchronize (native_linux.go:341-353). */
int manta_rocm_synchronize(MantaRocm* rt, char** err);

/* Replaces mantaCudaMemAlloc / mantaCudaMemFree (native_linux.go:285-311). */
int manta_rocm_malloc(MantaRocm* rt, void** out_dev, size_t bytes, char** err);
int manta_rocm_free(MantaRocm* rt, void* dev, char** err);

/* Replace mantaCudaMemcpyHtoD / DtoH (native_linux.go:313-339); download
 * synchronizes the stream first. */
int manta_rocm_upload(MantaRocm* rt, void* dst_dev, const void* src, size_t bytes, char** err);
int manta_rocm_download(MantaRocm* rt, void* dst, const void* src_dev, size_t bytes, char** err);

/* Counters in the spirit of matMulStatsSnapshot (native_linux.go:1474-1481). */
int manta_rocm_stats(const MantaRocm* rt, MantaRocmStats* out);

/* Per-kernel-family device timing.  With timing on, every launch is
 * bracketed by HIP events on the runtime's stream.  manta_rocm_timing
 * synchronizes, folds the finished events into totals and reports the launch
 * count and summed milliseconds of one family ("q8_scan", "q4_scan",
 * "topk_merge", "embed", ...; NULL = all), optionally clearing the totals.
 * Extends the reference's matmul counters (recordMatMulRun,
 * native_linux.go:1483-1497) with device time. */
int manta_rocm_set_timing(MantaRocm* rt, int on, char** err);
int manta_rocm_timing(MantaRocm* rt, const char* name, uint64_t* count, double* total_ms, int reset,
                      char** err);
/* Span timing: end = 0 records a start event on the runtime's stream, end = 1
 * a stop event; the second call waits for it and reports the milliseconds
 * between the two.  Times a run of launches with nothing recorded between
 * them (per-launch events add microseconds to short launches).  No
 * counterpart in the reference; a measurement aid beside manta_rocm_timing. */
int manta_rocm_span(MantaRocm* rt, int end, double* elapsed_ms, char** err);

/* ---- packing and candidate binding ------------------------------------ */

/* Host packers for f32 rows (the values a reference q8/q4 tensor carries).
 * Replace the per-tensor fake quantization grid (cuda quantizeBufferInPlace,
 * native_linux.go:2588-2619) with per-row / per-block packed storage. */
int manta_rocm_pack_q8_rows(const float* x, int64_t n, int64_t d, int8_t* codes, float* scales,
                            char** err);
int manta_rocm_pack_q4_blocks(const float* x, int64_t n, int64_t d, uint8_t* packed,
                              uint16_t* scales, char** err);

/* Exact repacking of the f32 values a reference q8 / q4 tensor carries
 * (bits 8 or 4) into q8 rows -- int8 codes + an f32 scale per row, bound with
 * manta_rocm_bind_q8_rows -- so that every value is the f32 product
 * code*scale.  *grid reports what was found: 2, the values lie on one
 * per-tensor symmetric grid, the reference's fakeQuantizeDataInPlace
 * (runtime/embedding_trainer.go:3738-3763; every row gets the tensor's
 * scale, codes in [-2^(bits-1)+1, 2^(bits-1)-1]); 1, each row lies on its own
 * grid of step maxabs_row/levels; 0, on neither, and the rows were
 * re-quantized per row to int8 (lossy, as manta_rocm_pack_q8_rows).  With
 * 2 or 1 the device scores equal the reference's on the original tensor.
 * No reference counterpart: replaces the per-tensor re-quantization at load
 * (cuda quantizeBufferInPlace, native_linux.go:2588-2619). */
int manta_rocm_pack_grid(const float* x, int64_t n, int64_t d, int bits, int8_t* codes, float* scales, int* grid,
                         char** err);

/* Make a device-resident candidate matrix from packed host arrays:
 * `sets` independent [n, d] matrices (sets == 1: one matrix shared by every
 * query, the [Q,D] x [N,D] form; sets == Q: one per query, the reference's
 * batched [Q,D] x [Q,N,D] form, tensor_ops.go:1511-1519).  Computes the
 * per-row norm constants.  Takes over the role of bindResidentMatMulParams
 * (cuda.go:129-169) for score inputs, which the reference re-uploads as f32
 * on every call (native_linux.go:1705-1714). */
int manta_rocm_bind_q8_rows(MantaRocm* rt, const int8_t* codes, const float* scales, int64_t sets,
                            int64_t n, int64_t d, MantaRocmCandidates** out, char** err);
int manta_rocm_bind_q4_blocks(MantaRocm* rt, const uint8_t* packed, const uint16_t* scales,
                              int64_t sets, int64_t n, int64_t d, MantaRocmCandidates** out,
                              char** err);
/* Bind the candidates of a packed container (manta_mll.h: QCOD / QSCL
 * sections opened with manta_mll_open) as one set, the bytes going to the
 * device as stored, with no f32 widening or re-quantisation.  Replaces the
 * load path ReadWeightFile -> decodeWeightFileFromMLLReader ->
 * decodeTensorEntry -> NewTensorQ4/Q8 of f32 values
 * (runtime/weight_file.go:93-104, 247-367) for candidate stores. */
int manta_rocm_bind_packed(MantaRocm* rt, const struct MantaMll* container, MantaRocmCandidates** out,
                           char** err);
/* Free a candidate set: its device memory (unless its runtime was destroyed
 * first, which released it) and the handle. */
void manta_rocm_unbind(MantaRocmCandidates* cands);
int manta_rocm_candidates_info(const MantaRocmCandidates* cands, int* format, int64_t* sets,
                               int64_t* n, int64_t* d);

/* ---- scoring ------------------------------------------------------------ */

/* Full score matrix.  queries_dev: f16 [nq, d]; out_scores_dev: f32 [nq, n].
 * op: MANTA_ROCM_DOT / COSINE / L2_DISTANCE, optionally with
 * MANTA_ROCM_QUANTIZED_QUERY.  Replaces runScoreKernel
 * (native_linux.go:1694-1732) and the host dotRows / cosineRows /
 * l2DistanceRows (tensor_ops.go:1366-1490) for packed candidates. */
int manta_rocm_score(MantaRocm* rt, const MantaRocmCandidates* cands, int op,
                     const uint16_t* queries_dev, int64_t nq, float* out_scores_dev, char** err);

/* Fused scoring + top-k: the score matrix is never written.  out_ids_dev
 * int32 [nq, k]; out_scores_dev f32 [nq, k] (may be NULL); out_acc_dev int64
 * [nq, k] (may be NULL): the exact integer accumulator of each selected row
 * (q8 candidates with MANTA_ROCM_QUANTIZED_QUERY only).  Replaces
 * launch_kernel(score) followed by the host topk step
 * (tensor_ops.go:119-135, 1523-1592).  Errors like topKTensor when k <= 0 or
 * k > n.  With reference scores the quantized-query scan ranks the rows, its
 * best few beyond k are rescored with the reference arithmetic, and the
 * error bounds between the two decide whether any other row could still
 * enter; a query where they cannot rule that out is rescanned with the
 * reference arithmetic, so the result is the reference's either way. */
int manta_rocm_score_topk(MantaRocm* rt, const MantaRocmCandidates* cands, int op, int order,
                          const uint16_t* queries_dev, int64_t nq, int64_t k,
                          int32_t* out_ids_dev, float* out_scores_dev, int64_t* out_acc_dev,
                          char** err);

/* manta_rocm_score_topk for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, semantics
 * and results as manta_rocm_score_topk (the same kernels), but the call makes
 * no device allocation and records no timing events: every scratch buffer
 * comes from a fixed device array of 32 MiB per GPU (minus 256 KiB of
 * tickets) that the library holds from the first runtime on that GPU until
 * the process ends.  Only the streaming scan (one query per workgroup) runs,
 * never the multi-query passes; a call that would need more scratch than the
 * array holds (about nq * (n / 16384 + 1) * k * 8 bytes, twice that and
 * nq * k * 16 more for reference scores) returns MANTA_ROCM_UNSUPPORTED.  The
 * array keeps the last call's contents; calls that overlap on one GPU race. */
int manta_rocm_score_topk_noalloc(MantaRocm* rt, const MantaRocmCandidates* cands, int op, int order,
                                  const uint16_t* queries_dev, int64_t nq, int64_t k, int32_t* out_ids_dev,
                                  float* out_scores_dev, int64_t* out_acc_dev, char** err);

/* The retrieval presets' last steps after top-k (compiler/compiler.go:539-570):
 * gather(candidate_ids, top), gather(docs, top) and pack_candidates
 * (tensor_ops.go:66-82, the pack holding ids, scores and docs, tensor.go:27-31),
 * on device and on the packed rows themselves.  top_dev: int32 [nq, k] row
 * indices (as manta_rocm_score_topk returns them); candidate_ids_dev: int64
 * [sets, n] or NULL; outputs: out_ids_dev int64 [nq, k] (skipped when
 * candidate_ids_dev is NULL), out_rows_dev [nq, k, row_bytes] with row_bytes =
 * d (q8) or d/2 (q4), out_scales_dev [nq, k, s] with s = 1 f32 (q8) or d/32
 * f16 (q4).  With sets == nq query q takes rows of set q.  The scores are the
 * top-k call's.  An index outside [0, n) zero-fills its slot and is reported
 * by the next synchronizing call as "gather index %d out of range". */
int manta_rocm_pack_candidates(MantaRocm* rt, const MantaRocmCandidates* cands, const int32_t* top_dev,
                               int64_t nq, int64_t k, const int64_t* candidate_ids_dev, int64_t* out_ids_dev,
                               void* out_rows_dev, void* out_scales_dev, char** err);

/* ---- encoder forward (examples/encoder_trainable_q8.manta) -------------- */

/* The weights of the one-layer encoder: q8 token rows ([vocab, d] int8 with
 * an f32 scale per row) and six q8 matrices with an f32 scale per output
 * column -- attn_q, attn_k, attn_v, attn_o [d, d], ffn_up [d, h],
 * projection [h, d].  Device pointers. */
typedef struct MantaRocmEncoderWeights {
    const int8_t* token_codes;
    const float* token_scales;
    const int8_t* codes[6];       /* attn_q, attn_k, attn_v, attn_o, ffn_up, projection */
    const float* col_scales[6];
} MantaRocmEncoderWeights;

/* embed_pooled_batch of examples/encoder_trainable_q8.manta:37-60 on the
 * device: gather + dequant, q/k/v projections, scores = q @ transpose(k)
 * per sequence (no scaling, every position attended, as the program
 * states), softmax, @ v, @ attn_o, layernorm(attended + hidden), ffn_up,
 * gelu, projection, layernorm(projected + attn_hidden), normalize, masked
 * mean pool; f16 out [b, d].  The steps are the reference's
 * gatherTensor / matmulTensor / transposeTensor / softmaxRows /
 * layerNormRows / geluTensor / normalizeRows / meanPoolMaskedTensor
 * (tensor_ops.go:751-1344), in f32.  Token ids out of range are reported by
 * the next synchronizing call, as manta_rocm_embed_pooled.  Replaces the
 * host execution of these steps (the CUDA backend offers only matmul and
 * normalize, cuda.go:270-299). */
int manta_rocm_encoder_pooled(MantaRocm* rt, const int32_t* tokens_dev, const int32_t* mask_dev, int64_t b,
                              int64_t t, const MantaRocmEncoderWeights* w, int64_t vocab, int64_t d, int64_t h,
                              uint16_t* out_dev, char** err);

/* The encoder block applied `layers` times (1..64) with the same weights,
 * each block's encoded output the next block's hidden input:
 * embed_pooled_batch of examples/encoder_trainable_q8x2.manta:9-50 is
 * layers = 2 (its manifest's encoder_repeats).  layers = 1 is
 * manta_rocm_encoder_pooled. */
int manta_rocm_encoder_pooled_layers(MantaRocm* rt, const int32_t* tokens_dev, const int32_t* mask_dev, int64_t b,
                                     int64_t t, const MantaRocmEncoderWeights* w, int64_t vocab, int64_t d,
                                     int64_t h, int64_t layers, uint16_t* out_dev, char** err);

/* top-k over an f32 score matrix [rows, cols] (rows == 1 is the rank-1
 * form).  Replaces topKTensor (tensor_ops.go:1523-1592). */
int manta_rocm_topk(MantaRocm* rt, const float* scores_dev, int64_t rows, int64_t cols, int64_t k,
                    int order, int32_t* out_ids_dev, float* out_values_dev, char** err);

/* ---- dense retrieval vectors ------------------------------------------- */

/* dotRetrievalVectors (runtime/retrieval_eval.go:651-661) on device: f32
 * queries [nq, qd] against rows [n, d] of f32 or f16 values (dtype
 * MANTA_ROCM_DENSE_F32 / _F16), the sum over min(qd, d) columns in f32,
 * product and sum rounded separately, in index order -- the reference's
 * scores bit for bit.  out_scores_dev f32 [nq, n]. */
int manta_rocm_dense_scores(MantaRocm* rt, const void* rows_dev, int dtype, int64_t n, int64_t d,
                            const float* queries_dev, int64_t nq, int64_t qd, float* out_scores_dev, char** err);

/* topRetrievalScores (retrieval_eval.go:586-623): the k best rows of each
 * query by (score desc, row asc) -- retrievalScoreBetter's (score desc, doc
 * ID asc) when the rows are stored in ascending doc-ID order, which is how a
 * host binds them (the Python wrapper sorts).  out_rows_dev int32 [nq, k],
 * out_scores_dev f32 [nq, k] (may be NULL).  k as manta_rocm_topk (the
 * reference's k <= 0 or k > n, "every doc", is the caller's k = n). */
int manta_rocm_dense_topk(MantaRocm* rt, const void* rows_dev, int dtype, int64_t n, int64_t d,
                          const float* queries_dev, int64_t nq, int64_t qd, int64_t k, int32_t* out_rows_dev,
                          float* out_scores_dev, char** err);

/* ---- embed pipeline ---------------------------------------------------- */

/* gatherTensor, f16 table [vocab, d] x int32 indices [nidx] -> f16
 * [nidx, d] (tensor_ops.go:794-877).  An out-of-range index leaves a zero
 * row and is reported by the next synchronizing call as "gather index %d out
 * of range". */
int manta_rocm_gather_rows_f16(MantaRocm* rt, const uint16_t* table_dev, int64_t vocab, int64_t d,
                               const int32_t* idx_dev, int64_t nidx, uint16_t* out_dev,
                               char** err);

/* matmulTensor [m,k] x [k,n] with f16 operands and f32 accumulation, f32
 * out (tensor_ops.go:981-1062; the CUDA path is cublasSgemm,
 * native_linux.go:509-549).  rhs is f16 or q8-per-column (proj_kind). */
int manta_rocm_matmul_f16(MantaRocm* rt, const uint16_t* lhs_dev, int64_t m, int64_t k,
                          const void* rhs_dev, int proj_kind, const float* col_scale_dev,
                          int64_t n, float* out_dev, char** err);

/* meanPoolMaskedTensor rank 3: f32 [b,t,c] with int32 mask [b,t] -> f32
 * [b,c] (tensor_ops.go:1210-1275). */
int manta_rocm_mean_pool_masked(MantaRocm* rt, const float* x_dev, const int32_t* mask_dev,
                                int64_t b, int64_t t, int64_t c, float* out_dev, char** err);

/* meanPoolTensor: f32 [b,t,c] -> f32 [b,c], every position counted, the f32
 * sum in position order divided by float32(t) (tensor_ops.go:1170-1208;
 * b == 1 is the rank-2 form). */
int manta_rocm_mean_pool(MantaRocm* rt, const float* x_dev, int64_t b, int64_t t, int64_t c, float* out_dev,
                         char** err);

/* normalizeRows: f32 [rows, cols] in place (tensor_ops.go:1114-1138, the
 * CUDA row-wise kernel at compiler/compiler.go:731-745). */
int manta_rocm_normalize_rows(MantaRocm* rt, float* x_dev, int64_t rows, int64_t cols,
                              char** err);

/* A projection weight in the layout the MFMA embed and matmul kernels read
 * (no counterpart in the reference: its weights are re-read per call).
 * proj_kind MANTA_ROCM_PROJ_F16 or MANTA_ROCM_PROJ_Q8_COL, [d, e]; writes
 * f16 [e, d] to out_dev (e*d*2 bytes) and the kind to pass with it
 * (MANTA_ROCM_PROJ_F16_T / _Q8_COL_T, same column scales) to *out_kind.
 * Prepared once when a weight is bound, it saves the per-call transpose
 * launch of the pipelined GEMMs.  Stream-ordered. */
int manta_rocm_prepare_projection(MantaRocm* rt, const void* proj_dev, int proj_kind, int64_t d, int64_t e,
                                  uint16_t* out_dev, int* out_kind, char** err);

/* The whole embed entry point in one fused launch sequence:
 * gather(table, tokens) -> @matmul(proj) -> mean_pool(mask) -> normalize,
 * f16 output [b, e].  mask_dev may be NULL (every position valid).  Token
 * ids are checked at every position, masked or not, like gatherTensor; an
 * out-of-range id is reported by the next synchronizing call
 * (manta_rocm_synchronize / manta_rocm_download) as
 * "gather index %d out of range".  Requires d % 8 == 0, e even (e % 4 for a
 * q8 projection) and e <= 4096, else MANTA_ROCM_UNSUPPORTED.  The [b,t,e] intermediate never reaches HBM.  Takes over
 * the host gather + cuBLAS + host mean_pool chain of
 * EmbeddingModel.EmbedBatch (runtime/embedding_model.go:422; stack in
 * tensor_ops.go:31-47, native_linux.go:3608-3670, tensor_ops.go:1210). */
int manta_rocm_embed_pooled(MantaRocm* rt, const int32_t* tokens_dev, const int32_t* mask_dev,
                            int64_t b, int64_t t, const uint16_t* table_dev, int64_t vocab,
                            int64_t d, const void* proj_dev, int proj_kind,
                            const float* col_scale_dev, int64_t e, uint16_t* out_dev,
                            char** err);

#ifdef __cplusplus
}
#endif
#endif
