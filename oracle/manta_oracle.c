/*
 * manta_oracle.c -- CPU oracle (test infrastructure only; see the header).
 *
 * Citations are to the reference tree odvcencio/manta:
 *   runtime/backend/tensor_ops.go   host executor ops
 *   runtime/retrieval_eval.go       bounded-heap host scorer
 *
 * Built with -ffp-contract=off: the Go compiler on amd64 (GOAMD64=v1, the
 * default) does not fuse a*b+c, so every f32 multiply and add is rounded on
 * its own, as here.
 */
#include "manta_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ f16 */

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-8f; /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e - 15u + 127u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) { /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477FF000u) { /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7C00u);
    }
    if (ax < 0x38800000u) { /* below 2^-14: f16 subnormal or zero */
        float a;
        memcpy(&a, &ax, 4);
        float s = a * 16777216.0f; /* exact scaling by 2^24 */
        uint32_t m = (uint32_t)nearbyintf(s); /* ties to even */
        return (uint16_t)(sign | m);
    }
    uint32_t e = (ax >> 23) - 127u + 15u;
    uint32_t mant = ax & 0x7FFFFFu;
    uint32_t h = (e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

void orc_f16_to_f32_array(const uint16_t* in, int64_t n, float* out) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(in[i]);
}

void orc_f32_to_f16_array(const float* in, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(in[i]);
}

/* ------------------------------------------- reference host executor ops */

static const float* docs_for(const float* docs, int64_t qi, int64_t rows,
                             int64_t cols, int docs_per_query) {
    return docs_per_query ? docs + qi * rows * cols : docs;
}

/* One row of dotRows, tensor_ops.go:1366-1396: f32 sum, sequential over
 * columns (each product and each sum rounded on its own). */
static float ref_dot_row(const float* q, const float* d, int64_t cols) {
    float sum = 0.0f;
    for (int64_t c = 0; c < cols; c++) sum += q[c] * d[c];
    return sum;
}

/* The query norm of cosineRows, tensor_ops.go:1404-1408 (f64, sequential). */
static double ref_query_norm(const float* q, int64_t cols) {
    double qn = 0.0;
    for (int64_t c = 0; c < cols; c++) {
        double v = (double)q[c];
        qn += v * v;
    }
    return qn;
}

/* One row of cosineRows, tensor_ops.go:1410-1425: f64 dot and row norm, 0
 * when the denominator is 0, narrowed to f32. */
static float ref_cosine_row(const float* q, double qn, const float* d, int64_t cols) {
    double dot = 0.0, dn = 0.0;
    for (int64_t c = 0; c < cols; c++) {
        double qq = (double)q[c];
        double dv = (double)d[c];
        dot += qq * dv;
        dn += dv * dv;
    }
    double denom = sqrt(qn) * sqrt(dn);
    return denom == 0.0 ? 0.0f : (float)(dot / denom);
}

/* One row of l2DistanceRows, tensor_ops.go:1464-1472: difference in f32,
 * squares and sum in f64, sqrt, narrowed. */
static float ref_l2_row(const float* q, const float* d, int64_t cols) {
    double sum = 0.0;
    for (int64_t c = 0; c < cols; c++) {
        float diff32 = q[c] - d[c];
        double diff = (double)diff32;
        sum += diff * diff;
    }
    return (float)sqrt(sum);
}

/* dotRows, tensor_ops.go:1366-1396. */
void orc_dot_rows(const float* q, const float* docs, int64_t nq, int64_t rows,
                  int64_t cols, int docs_per_query, float* out) {
    for (int64_t b = 0; b < nq; b++) {
        const float* qb = q + b * cols;
        const float* db = docs_for(docs, b, rows, cols, docs_per_query);
        for (int64_t r = 0; r < rows; r++) out[b * rows + r] = ref_dot_row(qb, db + r * cols, cols);
    }
}

/* cosineRows, tensor_ops.go:1398-1456. */
void orc_cosine_rows(const float* q, const float* docs, int64_t nq, int64_t rows,
                     int64_t cols, int docs_per_query, float* out) {
    for (int64_t b = 0; b < nq; b++) {
        const float* qb = q + b * cols;
        const float* db = docs_for(docs, b, rows, cols, docs_per_query);
        const double qn = ref_query_norm(qb, cols);
        for (int64_t r = 0; r < rows; r++) out[b * rows + r] = ref_cosine_row(qb, qn, db + r * cols, cols);
    }
}

/* l2DistanceRows, tensor_ops.go:1458-1490. */
void orc_l2_distance_rows(const float* q, const float* docs, int64_t nq,
                          int64_t rows, int64_t cols, int docs_per_query,
                          float* out) {
    for (int64_t b = 0; b < nq; b++) {
        const float* qb = q + b * cols;
        const float* db = docs_for(docs, b, rows, cols, docs_per_query);
        for (int64_t r = 0; r < rows; r++) out[b * rows + r] = ref_l2_row(qb, db + r * cols, cols);
    }
}

/* The f32 value a reference q8 / q4 tensor holds for a packed element: the
 * fake-quantization grid stores q*scale in f32
 * (runtime/embedding_trainer.go:3753-3762: data[i] = q * scale), so a q8
 * element is the f32 product code*scale and a q4 element code*f16scale
 * (exact: a 4-bit code times an 11-bit significand). */
static float q8_value(int8_t code, float scale) { return (float)code * scale; }

void orc_dequant_q8(const int8_t* codes, const float* scales, int64_t n, int64_t d, float* out) {
    for (int64_t r = 0; r < n; r++)
        for (int64_t c = 0; c < d; c++) out[r * d + c] = q8_value(codes[r * d + c], scales[r]);
}

static int q4_code(const uint8_t* row, int64_t c);

void orc_dequant_q4(const uint8_t* packed, const uint16_t* scales, int64_t n, int64_t d, float* out) {
    for (int64_t r = 0; r < n; r++)
        for (int64_t c = 0; c < d; c++)
            out[r * d + c] = (float)q4_code(packed + r * (d / 2), c) * orc_f16_to_f32(scales[r * (d / 32) + c / 32]);
}

/* fakeQuantizeDataInPlace, runtime/embedding_trainer.go:3738-3763: one
 * symmetric grid for the whole tensor, scale = maxAbs/levels (f32),
 * q = round(v/scale) (f32 division, half away from zero), clamped to
 * +-levels, value q*scale (f32); an all-zero tensor is left unchanged. */
void orc_fake_quantize(float* data, int64_t n, int bits) {
    if (bits <= 0 || n == 0) return;
    float maxabs = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        float a = (float)fabs((double)data[i]);
        if (a > maxabs) maxabs = a;
    }
    if (maxabs == 0.0f) return;
    const float levels = (float)((1 << (bits - 1)) - 1);
    if (levels <= 0.0f) return;
    const float scale = maxabs / levels;
    if (scale == 0.0f) return;
    for (int64_t i = 0; i < n; i++) {
        float q = (float)round((double)(data[i] / scale));
        if (q > levels) q = levels;
        if (q < -levels) q = -levels;
        data[i] = q * scale;
    }
}

/* dotRows / cosineRows / l2DistanceRows of f16 queries (widened to f32, as
 * the reference's f16 tensors are f32-backed, tensor.go:11-19) against the
 * dequantized values of packed candidates, row by row: the per-row loops
 * above on each dequantized row, so the bits equal those of the functions
 * above on a dequantized matrix. */
static void ref_score_rows(int op, const float* q32, const float* row, double qn, int64_t d, float* out) {
    if (op == ORC_DOT) *out = ref_dot_row(q32, row, d);
    else if (op == ORC_COSINE) *out = ref_cosine_row(q32, qn, row, d);
    else *out = ref_l2_row(q32, row, d);
}

void orc_ref_score_q8(int op, const uint16_t* queries, int64_t nq, const int8_t* codes,
                      const float* scales, int64_t sets, int64_t n, int64_t d, float* out) {
    float* q32 = (float*)malloc((size_t)d * sizeof(float));
    float* row = (float*)malloc((size_t)d * sizeof(float));
    for (int64_t b = 0; b < nq; b++) {
        const int64_t set = sets == 1 ? 0 : b;
        orc_f16_to_f32_array(queries + b * d, d, q32);
        const double qn = ref_query_norm(q32, d);
        for (int64_t r = 0; r < n; r++) {
            const int64_t gr = set * n + r;
            for (int64_t c = 0; c < d; c++) row[c] = q8_value(codes[gr * d + c], scales[gr]);
            ref_score_rows(op, q32, row, qn, d, out + b * n + r);
        }
    }
    free(q32);
    free(row);
}

void orc_ref_score_q4(int op, const uint16_t* queries, int64_t nq, const uint8_t* packed,
                      const uint16_t* scales, int64_t sets, int64_t n, int64_t d, float* out) {
    float* q32 = (float*)malloc((size_t)d * sizeof(float));
    float* row = (float*)malloc((size_t)d * sizeof(float));
    for (int64_t b = 0; b < nq; b++) {
        const int64_t set = sets == 1 ? 0 : b;
        orc_f16_to_f32_array(queries + b * d, d, q32);
        const double qn = ref_query_norm(q32, d);
        for (int64_t r = 0; r < n; r++) {
            const int64_t gr = set * n + r;
            orc_dequant_q4(packed + gr * (d / 2), scales + gr * (d / 32), 1, d, row);
            ref_score_rows(op, q32, row, qn, d, out + b * n + r);
        }
    }
    free(q32);
    free(row);
}

typedef struct {
    int64_t idx;
    float val;
} orc_pair;

/* Comparator of topKTensor (tensor_ops.go:1539-1551): value desc, index asc. */
static int cmp_largest(const void* pa, const void* pb) {
    const orc_pair* a = (const orc_pair*)pa;
    const orc_pair* b = (const orc_pair*)pb;
    if (a->val > b->val) return -1;
    if (a->val < b->val) return 1;
    if (a->idx < b->idx) return -1;
    if (a->idx > b->idx) return 1;
    return 0;
}

/* Smallest-k extension: value asc, index asc. */
static int cmp_smallest(const void* pa, const void* pb) {
    const orc_pair* a = (const orc_pair*)pa;
    const orc_pair* b = (const orc_pair*)pb;
    if (a->val < b->val) return -1;
    if (a->val > b->val) return 1;
    if (a->idx < b->idx) return -1;
    if (a->idx > b->idx) return 1;
    return 0;
}

/* topKTensor, tensor_ops.go:1523-1592 (rank-1 is nrows == 1). */
int orc_topk(const float* scores, int64_t nrows, int64_t ncols, int64_t k,
             int largest, int32_t* out_ids, char* msg, int msglen) {
    if (k <= 0 || k > ncols) {
        if (msg) {
            if (nrows == 1)
                snprintf(msg, (size_t)msglen,
                         "topk limit %lld out of range for %lld scores",
                         (long long)k, (long long)ncols);
            else
                snprintf(msg, (size_t)msglen,
                         "topk limit %lld out of range for row width %lld",
                         (long long)k, (long long)ncols);
        }
        return 1;
    }
    orc_pair* pairs = (orc_pair*)malloc((size_t)ncols * sizeof(orc_pair));
    if (!pairs) {
        if (msg) snprintf(msg, (size_t)msglen, "out of memory");
        return 1;
    }
    for (int64_t r = 0; r < nrows; r++) {
        for (int64_t c = 0; c < ncols; c++) {
            pairs[c].idx = c;
            pairs[c].val = scores[r * ncols + c];
        }
        qsort(pairs, (size_t)ncols, sizeof(orc_pair),
              largest ? cmp_largest : cmp_smallest);
        for (int64_t i = 0; i < k; i++) out_ids[r * k + i] = (int32_t)pairs[i].idx;
    }
    free(pairs);
    return 0;
}

/* gatherTensor rank-2 table (tensor_ops.go:794-877): row copies with a
 * bounds check per index. */
int orc_gather_rows(const float* table, int64_t rows, int64_t cols,
                    const int32_t* idx, int64_t nidx, float* out, char* msg,
                    int msglen) {
    for (int64_t i = 0; i < nidx; i++) {
        int32_t id = idx[i];
        if (id < 0 || (int64_t)id >= rows) {
            if (msg) snprintf(msg, (size_t)msglen, "gather index %d out of range", id);
            return 1;
        }
        memcpy(out + i * cols, table + (int64_t)id * cols, (size_t)cols * sizeof(float));
    }
    return 0;
}

/* matmulTensor [M,K]x[K,N], tensor_ops.go:993-1013 (the rank-3 x rank-2
 * form at :1015-1036 is the same loop over B*M rows). */
void orc_matmul(const float* lhs, const float* rhs, int64_t m, int64_t k,
                int64_t n, float* out) {
    for (int64_t i = 0; i < m; i++) {
        for (int64_t j = 0; j < n; j++) {
            float sum = 0.0f;
            for (int64_t kk = 0; kk < k; kk++) sum += lhs[i * k + kk] * rhs[kk * n + j];
            out[i * n + j] = sum;
        }
    }
}

/* meanPoolMaskedTensor rank-3, tensor_ops.go:1249-1271. */
void orc_mean_pool_masked(const float* x, const int32_t* mask, int64_t b,
                          int64_t t, int64_t c, float* out) {
    for (int64_t bi = 0; bi < b; bi++) {
        float* o = out + bi * c;
        for (int64_t j = 0; j < c; j++) o[j] = 0.0f;
        int64_t count = 0;
        for (int64_t r = 0; r < t; r++) {
            if (mask[bi * t + r] == 0) continue;
            count++;
            const float* row = x + (bi * t + r) * c;
            for (int64_t j = 0; j < c; j++) o[j] += row[j];
        }
        if (count == 0) continue;
        float inv = 1.0f / (float)count;
        for (int64_t j = 0; j < c; j++) o[j] *= inv;
    }
}

/* normalizeRows, tensor_ops.go:1114-1138: f64 sum of squares, f32 norm,
 * f32 division; a zero row is left unchanged. */
void orc_normalize_rows(float* x, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; r++) {
        double sum = 0.0;
        for (int64_t c = 0; c < cols; c++) {
            double v = (double)x[r * cols + c];
            sum += v * v;
        }
        float norm = (float)sqrt(sum);
        if (norm == 0.0f) continue;
        for (int64_t c = 0; c < cols; c++) x[r * cols + c] = x[r * cols + c] / norm;
    }
}

int orc_embed(const int32_t* tokens, const int32_t* mask, int64_t b, int64_t t,
              const uint16_t* table, int64_t vocab, int64_t d,
              const uint16_t* proj_f16, const int8_t* proj_codes,
              const float* proj_col_scale, int64_t e, uint16_t* out_f16,
              float* out_f32, char* msg, int msglen) {
    int64_t rows = b * t;
    float* g = (float*)malloc((size_t)(rows * d) * sizeof(float));
    float* w = (float*)malloc((size_t)(d * e) * sizeof(float));
    float* y = (float*)malloc((size_t)(rows * e) * sizeof(float));
    float* pooled = (float*)malloc((size_t)(b * e) * sizeof(float));
    int rc = 1;
    if (!g || !w || !y || !pooled) {
        if (msg) snprintf(msg, (size_t)msglen, "out of memory");
        goto done;
    }
    /* gather (f16 table values are carried as f32, tensor.go:11-12) */
    for (int64_t i = 0; i < rows; i++) {
        int32_t id = tokens[i];
        if (id < 0 || (int64_t)id >= vocab) {
            if (msg) snprintf(msg, (size_t)msglen, "gather index %d out of range", id);
            goto done;
        }
        orc_f16_to_f32_array(table + (int64_t)id * d, d, g + i * d);
    }
    if (proj_codes) {
        for (int64_t kk = 0; kk < d; kk++)
            for (int64_t j = 0; j < e; j++)
                w[kk * e + j] = (float)proj_codes[kk * e + j] * proj_col_scale[j];
    } else {
        orc_f16_to_f32_array(proj_f16, d * e, w);
    }
    orc_matmul(g, w, rows, d, e, y);
    orc_mean_pool_masked(y, mask, b, t, e, pooled);
    orc_normalize_rows(pooled, b, e);
    if (out_f32) memcpy(out_f32, pooled, (size_t)(b * e) * sizeof(float));
    if (out_f16) orc_f32_to_f16_array(pooled, b * e, out_f16);
    rc = 0;
done:
    free(g);
    free(w);
    free(y);
    free(pooled);
    return rc;
}

/* ---------------------------------------------- packed scoring contract */

void orc_pack_q8_rows(const float* x, int64_t n, int64_t d, int8_t* codes,
                      float* scales) {
    for (int64_t r = 0; r < n; r++) {
        const float* row = x + r * d;
        float maxabs = 0.0f;
        for (int64_t c = 0; c < d; c++) {
            float a = fabsf(row[c]);
            if (a > maxabs) maxabs = a;
        }
        if (maxabs == 0.0f) {
            memset(codes + r * d, 0, (size_t)d);
            scales[r] = 0.0f;
            continue;
        }
        for (int64_t c = 0; c < d; c++) {
            float v = row[c] * 127.0f;
            v = v / maxabs;
            float q = roundf(v);
            if (q > 127.0f) q = 127.0f;
            if (q < -127.0f) q = -127.0f;
            codes[r * d + c] = (int8_t)q;
        }
        scales[r] = maxabs / 127.0f;
    }
}

void orc_pack_q4_blocks(const float* x, int64_t n, int64_t d, uint8_t* packed,
                        uint16_t* scales) {
    int64_t nb = d / 32;
    for (int64_t r = 0; r < n; r++) {
        for (int64_t bk = 0; bk < nb; bk++) {
            const float* blk = x + r * d + bk * 32;
            float maxabs = 0.0f;
            for (int c = 0; c < 32; c++) {
                float a = fabsf(blk[c]);
                if (a > maxabs) maxabs = a;
            }
            int code[32];
            for (int c = 0; c < 32; c++) {
                if (maxabs == 0.0f) {
                    code[c] = 0;
                    continue;
                }
                float v = blk[c] * 7.0f;
                v = v / maxabs;
                float q = roundf(v);
                if (q > 7.0f) q = 7.0f;
                if (q < -7.0f) q = -7.0f;
                code[c] = (int)q;
            }
            uint8_t* dst = packed + r * (d / 2) + bk * 16;
            for (int j = 0; j < 16; j++)
                dst[j] = (uint8_t)((code[2 * j] & 0xF) | ((code[2 * j + 1] & 0xF) << 4));
            scales[r * nb + bk] = orc_f32_to_f16(maxabs == 0.0f ? 0.0f : maxabs / 7.0f);
        }
    }
}

static int q4_code(const uint8_t* row, int64_t c) {
    uint8_t byte = row[c >> 1];
    int v = (c & 1) ? (byte >> 4) : (byte & 0xF);
    return v >= 8 ? v - 16 : v;
}

void orc_q8_row_consts(const int8_t* codes, const float* scales, int64_t n,
                       int64_t d, float* dnorm, float* dd) {
    for (int64_t r = 0; r < n; r++) {
        int64_t ss = 0;
        for (int64_t c = 0; c < d; c++) {
            int64_t v = codes[r * d + c];
            ss += v * v;
        }
        double s = (double)scales[r];
        if (dnorm) dnorm[r] = (float)(sqrt((double)ss) * s);
        if (dd) dd[r] = (float)((double)ss * s * s);
    }
}

void orc_q4_row_consts(const uint8_t* packed, const uint16_t* scales,
                       int64_t n, int64_t d, float* dnorm, float* dd) {
    int64_t nb = d / 32;
    for (int64_t r = 0; r < n; r++) {
        const uint8_t* row = packed + r * (d / 2);
        double acc = 0.0;
        for (int64_t bk = 0; bk < nb; bk++) {
            int64_t ss = 0;
            for (int64_t c = bk * 32; c < bk * 32 + 32; c++) {
                int64_t v = q4_code(row, c);
                ss += v * v;
            }
            double s = (double)orc_f16_to_f32(scales[r * nb + bk]);
            acc += (s * s) * (double)ss;
        }
        if (dd) dd[r] = (float)acc;
        if (dnorm) dnorm[r] = (float)sqrt(acc);
    }
}

void orc_query_e8(const uint16_t* q, int64_t d, int8_t* codes, float* qmax_out) {
    float qmax = 1.0f;
    for (int64_t c = 0; c < d; c++) {
        float a = fabsf(orc_f16_to_f32(q[c]));
        if (a > qmax) qmax = a;
    }
    for (int64_t c = 0; c < d; c++) {
        float v = orc_f16_to_f32(q[c]) * 127.0f;
        v = v / qmax;
        float r = roundf(v);
        if (r > 127.0f) r = 127.0f;
        if (r < -127.0f) r = -127.0f;
        codes[c] = (int8_t)r;
    }
    *qmax_out = qmax;
}

void orc_query_e16(const uint16_t* q, int64_t d, int16_t* codes, float* qs,
                   float* qnorm, float* qq) {
    float qmax = 0.0f;
    for (int64_t c = 0; c < d; c++) {
        float a = fabsf(orc_f16_to_f32(q[c]));
        if (a > qmax) qmax = a;
    }
    if (qmax == 0.0f) {
        for (int64_t c = 0; c < d; c++) codes[c] = 0;
        *qs = 0.0f;
        *qnorm = 0.0f;
        *qq = 0.0f;
        return;
    }
    float inv = 32639.0f / qmax;
    int64_t ss = 0;
    for (int64_t c = 0; c < d; c++) {
        float v = orc_f16_to_f32(q[c]) * inv;
        float r = roundf(v);
        if (r > 32639.0f) r = 32639.0f;
        if (r < -32639.0f) r = -32639.0f;
        codes[c] = (int16_t)r;
        ss += (int64_t)codes[c] * (int64_t)codes[c];
    }
    float s = qmax / 32639.0f;
    *qs = s;
    *qnorm = (float)(sqrt((double)ss) * (double)s);
    *qq = (float)((double)ss * (double)s * (double)s);
}

static float finish_score(int op, float qd, float qnorm, float qq, float dnorm,
                          float dd) {
    if (op == ORC_DOT || op == ORC_DOT16) return qd;
    if (op == ORC_COSINE) {
        float den = qnorm * dnorm;
        return den == 0.0f ? 0.0f : qd / den;
    }
    float t = qq + dd;
    float dist2 = t - 2.0f * qd;
    if (dist2 < 0.0f) dist2 = 0.0f;
    return sqrtf(dist2);
}

void orc_score_q8(int op, const uint16_t* queries, int64_t nq,
                  const int8_t* codes, const float* scales, const float* dnorm,
                  const float* dd, int64_t sets, int64_t n, int64_t d,
                  float* out, int64_t* acc) {
    int8_t* c8 = (int8_t*)malloc((size_t)d);
    int16_t* c16 = (int16_t*)malloc((size_t)d * sizeof(int16_t));
    for (int64_t qi = 0; qi < nq; qi++) {
        int64_t set = sets == 1 ? 0 : qi;
        const int8_t* cs = codes + set * n * d;
        const float* sc = scales + set * n;
        const uint16_t* q = queries + qi * d;
        if (op == ORC_DOT) {
            float qmax;
            orc_query_e8(q, d, c8, &qmax);
            for (int64_t r = 0; r < n; r++) {
                int32_t a = 0;
                for (int64_t c = 0; c < d; c++) a += (int32_t)cs[r * d + c] * (int32_t)c8[c];
                float t = sc[r] * (float)a;
                t = t * qmax;
                out[qi * n + r] = t / 127.0f;
                if (acc) acc[qi * n + r] = a;
            }
        } else {
            float qs, qnorm, qq;
            orc_query_e16(q, d, c16, &qs, &qnorm, &qq);
            const float* dn = dnorm ? dnorm + set * n : NULL;
            const float* d2 = dd ? dd + set * n : NULL;
            for (int64_t r = 0; r < n; r++) {
                int64_t a = 0;
                for (int64_t c = 0; c < d; c++) a += (int64_t)cs[r * d + c] * (int64_t)c16[c];
                float sq = sc[r] * qs;
                float qd = sq * (float)a;
                out[qi * n + r] = finish_score(op, qd, qnorm, qq, dn ? dn[r] : 0.0f,
                                               d2 ? d2[r] : 0.0f);
                if (acc) acc[qi * n + r] = a;
            }
        }
    }
    free(c8);
    free(c16);
}

void orc_score_q4(int op, const uint16_t* queries, int64_t nq,
                  const uint8_t* packed, const uint16_t* scales,
                  const float* dnorm, const float* dd, int64_t sets, int64_t n,
                  int64_t d, float* out) {
    int64_t nb = d / 32;
    int16_t* c16 = (int16_t*)malloc((size_t)d * sizeof(int16_t));
    for (int64_t qi = 0; qi < nq; qi++) {
        int64_t set = sets == 1 ? 0 : qi;
        const uint8_t* ps = packed + set * n * (d / 2);
        const uint16_t* sc = scales + set * n * nb;
        float qs, qnorm, qq;
        orc_query_e16(queries + qi * d, d, c16, &qs, &qnorm, &qq);
        const float* dn = dnorm ? dnorm + set * n : NULL;
        const float* d2 = dd ? dd + set * n : NULL;
        for (int64_t r = 0; r < n; r++) {
            const uint8_t* row = ps + r * (d / 2);
            float dotf = 0.0f;
            for (int64_t bk = 0; bk < nb; bk++) {
                int32_t a = 0;
                for (int64_t c = bk * 32; c < bk * 32 + 32; c++) a += q4_code(row, c) * (int32_t)c16[c];
                dotf = fmaf(orc_f16_to_f32(sc[r * nb + bk]), (float)a, dotf);
            }
            float qd = dotf * qs;
            out[qi * n + r] = finish_score(op, qd, qnorm, qq, dn ? dn[r] : 0.0f,
                                           d2 ? d2[r] : 0.0f);
        }
    }
    free(c16);
}

/* ------------------------------------------------------ encoder ops */

/* layerNormRows, tensor_ops.go:1140-1168: f32 sequential mean and variance,
 * invStd = float32(1 / sqrt(float64(variance) + 1e-5)), no affine terms. */
void orc_layernorm_rows(float* x, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; r++) {
        float* row = x + r * cols;
        float mean = 0.0f;
        for (int64_t c = 0; c < cols; c++) mean += row[c];
        mean /= (float)cols;
        float variance = 0.0f;
        for (int64_t c = 0; c < cols; c++) {
            float centered = row[c] - mean;
            variance += centered * centered;
        }
        variance /= (float)cols;
        float inv_std = (float)(1.0 / sqrt((double)variance + 1e-5));
        for (int64_t c = 0; c < cols; c++) row[c] = (row[c] - mean) * inv_std;
    }
}

/* softmaxRows, tensor_ops.go:1303-1334: f32 max, exp of the f32 difference
 * in f64, f64 sum, f32 reciprocal of the sum, f32 products; a zero sum
 * leaves the exponentials. */
void orc_softmax_rows(float* x, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; r++) {
        float* row = x + r * cols;
        float max_v = row[0];
        for (int64_t c = 1; c < cols; c++)
            if (row[c] > max_v) max_v = row[c];
        double sum = 0.0;
        for (int64_t c = 0; c < cols; c++) {
            double ev = exp((double)(row[c] - max_v));
            row[c] = (float)ev;
            sum += ev;
        }
        if (sum == 0.0) continue;
        float inv = (float)(1.0 / sum);
        for (int64_t c = 0; c < cols; c++) row[c] *= inv;
    }
}

/* geluTensor, tensor_ops.go:1336-1344: the tanh approximation in f32 with
 * the tanh in f64. */
void orc_gelu(float* x, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        float v = x[i];
        float cubic = v * v * v;
        float inner = 0.7978845608f * (v + 0.044715f * cubic);
        x[i] = 0.5f * v * (1.0f + (float)tanh((double)inner));
    }
}

/* Batched [B,M,K] x [B,K,N] (matmulTensor rank 3 x rank 3,
 * tensor_ops.go:1037-1058): the [M,K]x[K,N] loop per batch. */
static void orc_matmul_batched(const float* lhs, const float* rhs, int64_t b, int64_t m, int64_t k,
                               int64_t n, float* out) {
    for (int64_t bi = 0; bi < b; bi++)
        orc_matmul(lhs + bi * m * k, rhs + bi * k * n, m, k, n, out + bi * m * n);
}

/* The encoder pipeline of examples/encoder_trainable_q8.manta:37-60
 * (embed_pooled_batch) over dequantized f32 values: gather, q/k/v
 * projections, scores = q @ transpose(k), softmax, @ v, @ attn_o, layernorm
 * of the residual sum, ffn_up, gelu, projection, layernorm of the residual
 * sum, normalize, masked mean pool.  out [b, d] f32. */
int orc_encoder_pooled(const int32_t* tokens, const int32_t* mask, int64_t b, int64_t t,
                       const float* table, int64_t vocab, int64_t d, const float* wq,
                       const float* wk, const float* wv, const float* wo, const float* wup,
                       const float* wproj, int64_t h, float* out, char* msg, int msglen) {
    return orc_encoder_pooled_layers(tokens, mask, b, t, table, vocab, d, wq, wk, wv, wo, wup, wproj, h, 1, out,
                                     msg, msglen);
}

/* The same with the encoder block applied `layers` times with shared
 * weights, each block's encoded output the next block's hidden input:
 * examples/encoder_trainable_q8x2.manta:9-50 is layers = 2 (the manifest's
 * encoder_repeats). */
int orc_encoder_pooled_layers(const int32_t* tokens, const int32_t* mask, int64_t b, int64_t t,
                              const float* table, int64_t vocab, int64_t d, const float* wq,
                              const float* wk, const float* wv, const float* wo, const float* wup,
                              const float* wproj, int64_t h, int64_t layers, float* out, char* msg,
                              int msglen) {
    const int64_t rows = b * t;
    float* hid = (float*)malloc((size_t)(rows * d) * sizeof(float));
    float* q = (float*)malloc((size_t)(rows * d) * sizeof(float));
    float* k = (float*)malloc((size_t)(rows * d) * sizeof(float));
    float* v = (float*)malloc((size_t)(rows * d) * sizeof(float));
    float* kt = (float*)malloc((size_t)(rows * d) * sizeof(float));
    float* s = (float*)malloc((size_t)(b * t * t) * sizeof(float));
    float* mixed = (float*)malloc((size_t)(rows * d) * sizeof(float));
    float* att = (float*)malloc((size_t)(rows * d) * sizeof(float));
    float* f = (float*)malloc((size_t)(rows * h) * sizeof(float));
    int rc = 1;
    if (!hid || !q || !k || !v || !kt || !s || !mixed || !att || !f) {
        if (msg) snprintf(msg, (size_t)msglen, "out of memory");
        goto done;
    }
    if (orc_gather_rows(table, vocab, d, tokens, rows, hid, msg, msglen)) goto done;
    for (int64_t layer = 0; layer < layers; layer++) {
    if (layer > 0) memcpy(hid, q, (size_t)(rows * d) * sizeof(float)); /* encoded -> hidden */
    orc_matmul(hid, wq, rows, d, d, q);
    orc_matmul(hid, wk, rows, d, d, k);
    orc_matmul(hid, wv, rows, d, d, v);
    for (int64_t bi = 0; bi < b; bi++) /* transpose of each [t, d] block */
        for (int64_t r = 0; r < t; r++)
            for (int64_t c = 0; c < d; c++) kt[bi * d * t + c * t + r] = k[bi * t * d + r * d + c];
    orc_matmul_batched(q, kt, b, t, d, t, s);
    orc_softmax_rows(s, b * t, t);
    orc_matmul_batched(s, v, b, t, t, d, mixed);
    orc_matmul(mixed, wo, rows, d, d, att);
    for (int64_t i = 0; i < rows * d; i++) att[i] = att[i] + hid[i]; /* attended + hidden */
    orc_layernorm_rows(att, rows, d);                                /* attn_hidden */
    orc_matmul(att, wup, rows, d, h, f);
    orc_gelu(f, rows * h);
    orc_matmul(f, wproj, rows, h, d, q);                             /* projected */
    for (int64_t i = 0; i < rows * d; i++) q[i] = q[i] + att[i];     /* + attn_hidden */
    orc_layernorm_rows(q, rows, d);                                  /* encoded */
    }
    orc_normalize_rows(q, rows, d);
    orc_mean_pool_masked(q, mask, b, t, d, out);
    rc = 0;
done:
    free(hid); free(q); free(k); free(v); free(kt); free(s); free(mixed); free(att); free(f);
    return rc;
}

/* ---- topRetrievalScores (runtime/retrieval_eval.go:586-661) ------------ */

typedef struct {
    float score;
    const char* id;
    int64_t pos;
} retrieval_doc;

/* retrievalScoreBetter, retrieval_eval.go:615-623. */
static int retrieval_better(const retrieval_doc* a, const retrieval_doc* b) {
    if (a->score > b->score) return 1;
    if (a->score < b->score) return 0;
    return strcmp(a->id, b->id) < 0;
}

/* container/heap over retrievalScoreHeap, whose Less(i, j) is
 * better(h[j], h[i]): the root is the worst kept doc. */
static int heap_less(const retrieval_doc* h, int64_t i, int64_t j) { return retrieval_better(&h[j], &h[i]); }

static void heap_up(retrieval_doc* h, int64_t j) {
    while (j > 0) {
        int64_t i = (j - 1) / 2;
        if (i == j || !heap_less(h, j, i)) break;
        retrieval_doc t = h[i];
        h[i] = h[j];
        h[j] = t;
        j = i;
    }
}

static void heap_down(retrieval_doc* h, int64_t i0, int64_t n) {
    int64_t i = i0;
    for (;;) {
        int64_t j1 = 2 * i + 1;
        if (j1 >= n || j1 < 0) break;
        int64_t j = j1;
        if (j1 + 1 < n && heap_less(h, j1 + 1, j1)) j = j1 + 1;
        if (!heap_less(h, j, i)) break;
        retrieval_doc t = h[i];
        h[i] = h[j];
        h[j] = t;
        i = j;
    }
}

static int retrieval_cmp(const void* pa, const void* pb) {
    const retrieval_doc* a = (const retrieval_doc*)pa;
    const retrieval_doc* b = (const retrieval_doc*)pb;
    if (retrieval_better(a, b)) return -1;
    if (retrieval_better(b, a)) return 1;
    return 0;
}

int64_t orc_top_retrieval_scores(const float* query, int64_t qd, const float* docs, int64_t n, int64_t d,
                                 const char* const* ids, int64_t top_k, int64_t* out_pos, float* out_scores) {
    if (top_k <= 0 || top_k > n) top_k = n;
    retrieval_doc* h = (retrieval_doc*)malloc((size_t)(top_k > 0 ? top_k : 1) * sizeof(retrieval_doc));
    const int64_t len = qd < d ? qd : d;
    int64_t cnt = 0;
    for (int64_t r = 0; r < n; r++) {
        retrieval_doc s = {ref_dot_row(query, docs + r * d, len), ids[r], r};
        if (cnt < top_k) {
            h[cnt] = s; /* heap.Push */
            heap_up(h, cnt);
            cnt++;
            continue;
        }
        if (retrieval_better(&s, &h[0])) {
            h[0] = s; /* heap.Fix(&h, 0) */
            heap_down(h, 0, cnt);
        }
    }
    qsort(h, (size_t)cnt, sizeof(retrieval_doc), retrieval_cmp);
    for (int64_t i = 0; i < cnt; i++) {
        out_pos[i] = h[i].pos;
        out_scores[i] = h[i].score;
    }
    free(h);
    return cnt;
}
