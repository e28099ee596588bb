/*
 * manta_oracle.h -- CPU oracle for the retrieval hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this code.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker / CPU baseline.
 *
 * Two groups of functions:
 *
 *  1. Restatements of the reference's host executor (Go, odvcencio/manta,
 *     runtime/backend/tensor_ops.go).  Same accumulation types and the same
 *     order of operations as the Go loops, so for identical inputs they give
 *     the bits the Go host path gives.  Each function cites the Go lines.
 *
 *  2. The packed q8/q4 scoring contract.  The reference has no packed layout
 *     (q4/q8 are f32-backed fake-quantized tensors, tensor.go:49-71); the
 *     packed formats and the integer/f32 scoring formulas below are defined by
 *     this repository and implemented here as
 *     plain loops.  The GPU kernels must reproduce them bit for bit.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no FMA contraction).
 */
#ifndef MANTA_ORACLE_H
#define MANTA_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ORC_DOT16: the q8 dot with E16 query codes (qd below), the scan score the
 * device ranks reference-semantics dot top-k by. */
enum { ORC_DOT = 0, ORC_COSINE = 1, ORC_L2 = 2, ORC_DOT16 = 3 };

/* IEEE binary16 <-> binary32 (round to nearest even). */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
void orc_f16_to_f32_array(const uint16_t* in, int64_t n, float* out);
void orc_f32_to_f16_array(const float* in, int64_t n, uint16_t* out);

/* ---- 1. reference host executor restatements ------------------------- */

/* Score layout (tensor_ops.go:1499-1521): docs_per_query != 0 means the
 * reference's batched form [Q,D] x [Q,N,D]; 0 with nq == 1 is [D] x [N,D];
 * 0 with nq > 1 is the shared-candidate extension [Q,D] x [N,D] (each query
 * against the same docs, same per-row arithmetic). out is [nq, rows]. */
void orc_dot_rows(const float* q, const float* docs, int64_t nq, int64_t rows,
                  int64_t cols, int docs_per_query, float* out);
void orc_cosine_rows(const float* q, const float* docs, int64_t nq, int64_t rows,
                     int64_t cols, int docs_per_query, float* out);
void orc_l2_distance_rows(const float* q, const float* docs, int64_t nq,
                          int64_t rows, int64_t cols, int docs_per_query,
                          float* out);

/* topKTensor (tensor_ops.go:1523-1592): per row, full sort by (value desc,
 * index asc) and emit the first k indices.  largest == 0 is the smallest-k
 * extension: (value asc, index asc).  Returns 0, or 1 with msg filled when
 * k <= 0 || k > ncols (same condition and wording as the Go error). */
int orc_topk(const float* scores, int64_t nrows, int64_t ncols, int64_t k,
             int largest, int32_t* out_ids, char* msg, int msglen);

/* gatherTensor, rank-2 table x rank-1/2 indices (tensor_ops.go:794-877):
 * out[i,:] = table[idx[i],:]; error on an out-of-range index. */
int orc_gather_rows(const float* table, int64_t rows, int64_t cols,
                    const int32_t* idx, int64_t nidx, float* out, char* msg,
                    int msglen);

/* matmulTensor [M,K]x[K,N] (tensor_ops.go:993-1013), f32 sequential k loop. */
void orc_matmul(const float* lhs, const float* rhs, int64_t m, int64_t k,
                int64_t n, float* out);

/* meanPoolMaskedTensor rank-3 (tensor_ops.go:1249-1271). */
void orc_mean_pool_masked(const float* x, const int32_t* mask, int64_t b,
                          int64_t t, int64_t c, float* out);

/* normalizeRows (tensor_ops.go:1114-1138), in place. */
void orc_normalize_rows(float* x, int64_t rows, int64_t cols);

/* The embed entry point of BASELINE configs 1 and 4:
 * gather -> @matmul -> masked mean_pool -> normalize, composed from the
 * functions above exactly as ExecuteSymbolic walks the steps.  table is f16
 * [V,D]; proj is either f16 [D,E] (proj_codes == NULL) or q8 codes [D,E] with
 * a per-output-column f32 scale (dequantized to f32 as code*scale, the value
 * a q8 tensor carries in the reference).  Output f16 [B,E]. */
int orc_embed(const int32_t* tokens, const int32_t* mask, int64_t b, int64_t t,
              const uint16_t* table, int64_t vocab, int64_t d,
              const uint16_t* proj_f16, const int8_t* proj_codes,
              const float* proj_col_scale, int64_t e, uint16_t* out_f16,
              float* out_f32, char* msg, int msglen);

/* The f32 values a reference q8 / q4 tensor carries for packed elements
 * (code*scale in f32; q4: code*f16scale, exact).  out [n, d]. */
void orc_dequant_q8(const int8_t* codes, const float* scales, int64_t n,
                    int64_t d, float* out);
void orc_dequant_q4(const uint8_t* packed, const uint16_t* scales, int64_t n,
                    int64_t d, float* out);

/* dotRows / cosineRows / l2DistanceRows (op ORC_*) of f16 queries [nq, d]
 * (widened to f32) against the dequantized rows of packed candidates
 * [sets, n, d] (sets 1: shared; sets nq: one set per query).  Bit-identical
 * to the functions above applied to orc_dequant_* output.  out [nq, n]. */
void orc_ref_score_q8(int op, const uint16_t* queries, int64_t nq,
                      const int8_t* codes, const float* scales, int64_t sets,
                      int64_t n, int64_t d, float* out);
void orc_ref_score_q4(int op, const uint16_t* queries, int64_t nq,
                      const uint8_t* packed, const uint16_t* scales,
                      int64_t sets, int64_t n, int64_t d, float* out);

/* fakeQuantizeDataInPlace (runtime/embedding_trainer.go:3738-3763): the
 * reference's per-tensor symmetric grid, in place. */
void orc_fake_quantize(float* data, int64_t n, int bits);

/* The encoder of examples/encoder_trainable_q8.manta (one block) and
 * encoder_trainable_q8x2.manta (the block applied `layers` times with
 * shared weights) over dequantized f32 weights; out f32 [b, d]. */
int orc_encoder_pooled(const int32_t* tokens, const int32_t* mask, int64_t b, int64_t t, const float* table,
                       int64_t vocab, int64_t d, const float* wq, const float* wk, const float* wv, const float* wo,
                       const float* wup, const float* wproj, int64_t h, float* out, char* msg, int msglen);
int orc_encoder_pooled_layers(const int32_t* tokens, const int32_t* mask, int64_t b, int64_t t,
                              const float* table, int64_t vocab, int64_t d, const float* wq, const float* wk,
                              const float* wv, const float* wo, const float* wup, const float* wproj, int64_t h,
                              int64_t layers, float* out, char* msg, int msglen);

/* topRetrievalScores + dotRetrievalVectors (runtime/retrieval_eval.go:
 * 586-661) for one f32 query [qd] against n f32 doc vectors [n, d] with
 * NUL-terminated doc ids: the bounded heap of the top_k (top_k <= 0 or
 * > n: all n) by retrievalScoreBetter (score desc, then id asc, bytewise),
 * then sorted; the dot runs over min(qd, d) columns.  Writes the chosen
 * docs' positions and scores in rank order; returns how many. */
int64_t orc_top_retrieval_scores(const float* query, int64_t qd, const float* docs, int64_t n, int64_t d,
                                 const char* const* ids, int64_t top_k, int64_t* out_pos, float* out_scores);

/* ---- 2. packed scoring contract (defined by this repository) ---------- */

/* q8 rows: code = clamp(round((x*127)/maxabs), -127, 127), scale =
 * maxabs/127 (all f32, round = half away from zero); all-zero row -> codes
 * 0, scale 0. */
void orc_pack_q8_rows(const float* x, int64_t n, int64_t d, int8_t* codes,
                      float* scales);
/* q4 blocks of 32 along D: code = clamp(round((x*7)/maxabs), -7, 7); two
 * codes per byte, low nibble first (two's complement nibbles); f16 scale =
 * f16(maxabs/7). */
void orc_pack_q4_blocks(const float* x, int64_t n, int64_t d, uint8_t* packed,
                        uint16_t* scales);

/* Per-row constants the bind step stores: dnorm = |row| and dd = |row|^2
 * of the dequantized row, f64 then narrowed. */
void orc_q8_row_consts(const int8_t* codes, const float* scales, int64_t n,
                       int64_t d, float* dnorm, float* dd);
void orc_q4_row_consts(const uint8_t* packed, const uint16_t* scales,
                       int64_t n, int64_t d, float* dnorm, float* dd);

/* Query encodings.
 * E8  (q8 dot): qmax = max(1, maxabs(q)); code = clamp(round((q*127)/qmax)).
 * E16 (all else): qmax = maxabs(q); code = clamp(round(q*(32639/qmax)),
 *     +-32639); qs = qmax/32639; qnorm = sqrt(sum code^2)*qs and
 *     qq = sum code^2 * qs^2 (f64, narrowed). */
void orc_query_e8(const uint16_t* q, int64_t d, int8_t* codes, float* qmax);
void orc_query_e16(const uint16_t* q, int64_t d, int16_t* codes, float* qs,
                   float* qnorm, float* qq);

/* Packed scoring.  queries f16 [nq,d]; candidates [sets,n,d] where sets is 1
 * (shared by every query) or nq (one candidate set per query, the
 * reference's batched layout).  out [nq,n].  acc (optional, may be NULL):
 * q8 dot -> int32 sum(code*qcode) widened to int64; q8 cosine/l2 -> int64
 * sum(code*qcode16); q4 -> unused. */
void orc_score_q8(int op, const uint16_t* queries, int64_t nq,
                  const int8_t* codes, const float* scales, const float* dnorm,
                  const float* dd, int64_t sets, int64_t n, int64_t d,
                  float* out, int64_t* acc);
void orc_score_q4(int op, const uint16_t* queries, int64_t nq,
                  const uint8_t* packed, const uint16_t* scales,
                  const float* dnorm, const float* dd, int64_t sets, int64_t n,
                  int64_t d, float* out);

/* ---- 3. bench.py's all-core CPU baseline (fair_cpu.c) ---------------- */

/* Quantized-query scores on the packed data (same formulas as above),
 * bounded heaps, rows split over `threads` OpenMP threads; candidates shared
 * by every query.  out_vals may be NULL. */
void orc_fair_q8_topk(int op, const uint16_t* queries, int64_t nq,
                      const int8_t* codes, const float* scales,
                      const float* dnorm, const float* dd, int64_t n, int64_t d,
                      int64_t k, int smallest, int threads, int32_t* out_ids,
                      float* out_vals);
void orc_fair_q4_topk(int op, const uint16_t* queries, int64_t nq,
                      const uint8_t* packed, const uint16_t* scales,
                      const float* dnorm, const float* dd, int64_t n, int64_t d,
                      int64_t k, int smallest, int threads, int32_t* out_ids,
                      float* out_vals);
/* The embed pipeline in f32 with sequences over threads; out f32 [b, e]. */
void orc_fair_embed(const int32_t* tokens, const int32_t* mask, int64_t b,
                    int64_t t, const uint16_t* table, int64_t vocab, int64_t d,
                    const uint16_t* proj_f16, const int8_t* proj_codes,
                    const float* col_scale, int64_t e, int threads, float* out);

#ifdef __cplusplus
}
#endif
#endif
