/*
 * fair_cpu.c -- the "fair CPU" baseline of bench.py (test infrastructure
 * only: nothing in the shipped library links it).
 *
 * The reference's host path (manta_oracle.c) widens q8/q4 tensors to f32 and
 * sorts every score; a CPU implementation written for throughput would not.
 * This one computes the same quantized-query scores as the GPU scans
 * (E8 q8 dot, E16 cosine / l2 / q4; see manta_oracle.h) on the packed
 * int8 / nibble data, keeps a bounded heap of the k best per thread, and
 * splits each query's rows over all threads (OpenMP).  Built -O3 -mavx2 so
 * the integer dot loops vectorize.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "manta_oracle.h"

#ifdef _OPENMP
#include <omp.h>
#endif

typedef struct {
    float v;
    int32_t i;
} entry;

/* a before b in the output order: value desc (asc for smallest), index asc */
static int better(entry a, entry b, int smallest) {
    if (a.v != b.v) return smallest ? a.v < b.v : a.v > b.v;
    return a.i < b.i;
}

/* Bounded heap of the k best: h[0] is the worst kept. */
static void heap_offer(entry* h, int* cnt, int k, entry e, int smallest) {
    if (*cnt < k) {
        int j = (*cnt)++;
        h[j] = e;
        while (j > 0) {
            int p = (j - 1) / 2;
            if (!better(h[p], h[j], smallest)) break;
            entry t = h[p];
            h[p] = h[j];
            h[j] = t;
            j = p;
        }
        return;
    }
    if (!better(e, h[0], smallest)) return;
    h[0] = e;
    int j = 0;
    for (;;) {
        int l = 2 * j + 1, r = l + 1, w = j;
        if (l < k && better(h[w], h[l], smallest)) w = l;
        if (r < k && better(h[w], h[r], smallest)) w = r;
        if (w == j) break;
        entry t = h[w];
        h[w] = h[j];
        h[j] = t;
        j = w;
    }
}

static int cmp_desc;
static int entry_cmp(const void* pa, const void* pb) {
    const entry* a = (const entry*)pa;
    const entry* b = (const entry*)pb;
    if (better(*a, *b, cmp_desc)) return -1;
    if (better(*b, *a, cmp_desc)) return 1;
    return 0;
}

static float finish(int op, float qd, float qn, float qq, float dn, float d2) {
    if (op == ORC_DOT || op == ORC_DOT16) return qd;
    if (op == ORC_COSINE) {
        float den = qn * dn;
        return den == 0.0f ? 0.0f : qd / den;
    }
    float t = qq + d2;
    float dist2 = t - 2.0f * qd;
    if (dist2 < 0.0f) dist2 = 0.0f;
    return sqrtf(dist2);
}

/* Merge per-thread heaps into the sorted k best of one query. */
static void merge_out(entry* heaps, const int* cnts, int nt, int k, int smallest, int32_t* ids, float* vals) {
    entry* all = (entry*)malloc((size_t)nt * k * sizeof(entry));
    int m = 0;
    for (int t = 0; t < nt; t++)
        for (int j = 0; j < cnts[t]; j++) all[m++] = heaps[(size_t)t * k + j];
    cmp_desc = smallest;
    qsort(all, (size_t)m, sizeof(entry), entry_cmp);
    for (int j = 0; j < k; j++) {
        ids[j] = j < m ? all[j].i : -1;
        if (vals) vals[j] = j < m ? all[j].v : 0.0f;
    }
    free(all);
}

/* q8 rows [n, d] shared by every query; op ORC_DOT (E8) or the E16 ops.
 * int32 accumulation: exact for d <= 512 with E16 codes. */
void orc_fair_q8_topk(int op, const uint16_t* queries, int64_t nq, const int8_t* codes, const float* scales,
                      const float* dnorm, const float* dd, int64_t n, int64_t d, int64_t k, int smallest,
                      int threads, int32_t* out_ids, float* out_vals) {
    entry* heaps = (entry*)malloc((size_t)threads * k * sizeof(entry));
    int* cnts = (int*)calloc((size_t)threads, sizeof(int));
    int16_t* qc = (int16_t*)malloc((size_t)d * sizeof(int16_t));
    int8_t* q8 = (int8_t*)malloc((size_t)d);
    for (int64_t qi = 0; qi < nq; qi++) {
        float qmax = 0, qs = 0, qn = 0, qq = 0;
        if (op == ORC_DOT) {
            orc_query_e8(queries + qi * d, d, q8, &qmax);
            for (int64_t c = 0; c < d; c++) qc[c] = q8[c];
        } else {
            orc_query_e16(queries + qi * d, d, qc, &qs, &qn, &qq);
        }
        memset(cnts, 0, (size_t)threads * sizeof(int));
#pragma omp parallel num_threads(threads)
        {
            int t = 0, nt = 1;
#ifdef _OPENMP
            t = omp_get_thread_num();
            nt = omp_get_num_threads();
#endif
            int64_t per = (n + nt - 1) / nt, r0 = t * per, r1 = r0 + per < n ? r0 + per : n;
            entry* h = heaps + (size_t)t * k;
            int cnt = 0;
            for (int64_t r = r0; r < r1; r++) {
                const int8_t* row = codes + r * d;
                int32_t a = 0;
                for (int64_t c = 0; c < d; c++) a += (int32_t)row[c] * (int32_t)qc[c];
                float s;
                if (op == ORC_DOT) {
                    float x = scales[r] * (float)a;
                    x = x * qmax;
                    s = x / 127.0f;
                } else {
                    float qd = (scales[r] * qs) * (float)a;
                    s = finish(op, qd, qn, qq, dnorm ? dnorm[r] : 0.0f, dd ? dd[r] : 0.0f);
                }
                entry e = {s, (int32_t)r};
                heap_offer(h, &cnt, (int)k, e, smallest);
            }
            cnts[t] = cnt;
        }
        merge_out(heaps, cnts, threads, (int)k, smallest, out_ids + qi * k, out_vals ? out_vals + qi * k : NULL);
    }
    free(heaps);
    free(cnts);
    free(qc);
    free(q8);
}

/* q4 blocks [n, d/2] + f16 scales [n, d/32] shared by every query (E16). */
void orc_fair_q4_topk(int op, const uint16_t* queries, int64_t nq, const uint8_t* packed, const uint16_t* scales,
                      const float* dnorm, const float* dd, int64_t n, int64_t d, int64_t k, int smallest,
                      int threads, int32_t* out_ids, float* out_vals) {
    const int64_t nb = d / 32;
    entry* heaps = (entry*)malloc((size_t)threads * k * sizeof(entry));
    int* cnts = (int*)calloc((size_t)threads, sizeof(int));
    int16_t* qc = (int16_t*)malloc((size_t)d * sizeof(int16_t));
    float* sf = (float*)malloc((size_t)n * nb * sizeof(float));
    for (int64_t i = 0; i < n * nb; i++) sf[i] = orc_f16_to_f32(scales[i]);
    for (int64_t qi = 0; qi < nq; qi++) {
        float qs, qn, qq;
        orc_query_e16(queries + qi * d, d, qc, &qs, &qn, &qq);
        memset(cnts, 0, (size_t)threads * sizeof(int));
#pragma omp parallel num_threads(threads)
        {
            int t = 0, nt = 1;
#ifdef _OPENMP
            t = omp_get_thread_num();
            nt = omp_get_num_threads();
#endif
            int64_t per = (n + nt - 1) / nt, r0 = t * per, r1 = r0 + per < n ? r0 + per : n;
            entry* h = heaps + (size_t)t * k;
            int cnt = 0;
            int16_t lo[32], hi[32];
            for (int64_t r = r0; r < r1; r++) {
                const uint8_t* row = packed + r * (d / 2);
                float dotf = 0.0f;
                for (int64_t b = 0; b < nb; b++) {
                    for (int j = 0; j < 16; j++) {
                        uint8_t byte = row[b * 16 + j];
                        lo[j] = (int16_t)((int8_t)(byte << 4) >> 4);
                        hi[j] = (int16_t)((int8_t)byte >> 4);
                    }
                    int32_t a = 0;
                    for (int j = 0; j < 16; j++)
                        a += lo[j] * (int32_t)qc[b * 32 + 2 * j] + hi[j] * (int32_t)qc[b * 32 + 2 * j + 1];
                    dotf = fmaf(sf[r * nb + b], (float)a, dotf);
                }
                float s = finish(op, dotf * qs, qn, qq, dnorm ? dnorm[r] : 0.0f, dd ? dd[r] : 0.0f);
                entry e = {s, (int32_t)r};
                heap_offer(h, &cnt, (int)k, e, smallest);
            }
            cnts[t] = cnt;
        }
        merge_out(heaps, cnts, threads, (int)k, smallest, out_ids + qi * k, out_vals ? out_vals + qi * k : NULL);
    }
    free(heaps);
    free(cnts);
    free(qc);
    free(sf);
}

/* The embed pipeline (gather -> matmul -> masked mean_pool -> normalize)
 * with sequences split over threads; f32 throughout, the matmul as
 * row x projection with the projection widened to f32 once. */
void orc_fair_embed(const int32_t* tokens, const int32_t* mask, int64_t b, int64_t t, const uint16_t* table,
                    int64_t vocab, int64_t d, const uint16_t* proj_f16, const int8_t* proj_codes,
                    const float* col_scale, int64_t e, int threads, float* out) {
    float* w = (float*)malloc((size_t)d * e * sizeof(float));
    for (int64_t i = 0; i < d; i++)
        for (int64_t j = 0; j < e; j++)
            w[i * e + j] = proj_codes ? (float)proj_codes[i * e + j] * col_scale[j] : orc_f16_to_f32(proj_f16[i * e + j]);
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
    for (int64_t s = 0; s < b; s++) {
        float* acc = (float*)calloc((size_t)e, sizeof(float));
        float* x = (float*)malloc((size_t)d * sizeof(float));
        float* y = (float*)malloc((size_t)e * sizeof(float));
        int64_t count = 0;
        for (int64_t p = 0; p < t; p++) {
            if (mask && mask[s * t + p] == 0) continue;
            int32_t id = tokens[s * t + p];
            if (id < 0 || id >= vocab) continue;
            for (int64_t c = 0; c < d; c++) x[c] = orc_f16_to_f32(table[(int64_t)id * d + c]);
            for (int64_t j = 0; j < e; j++) y[j] = 0.0f;
            for (int64_t c = 0; c < d; c++) {
                const float xc = x[c];
                const float* wr = w + c * e;
                for (int64_t j = 0; j < e; j++) y[j] += xc * wr[j];
            }
            for (int64_t j = 0; j < e; j++) acc[j] += y[j];
            count++;
        }
        float inv = count ? 1.0f / (float)count : 0.0f;
        double ss = 0.0;
        for (int64_t j = 0; j < e; j++) {
            acc[j] *= inv;
            ss += (double)acc[j] * acc[j];
        }
        float nrm = (float)sqrt(ss);
        for (int64_t j = 0; j < e; j++) out[s * e + j] = nrm > 0.0f ? acc[j] / nrm : acc[j];
        free(acc);
        free(x);
        free(y);
    }
    free(w);
}
