/*
 * kvhp_oracle.c -- CPU restatement of the serving-engine KV-cache hot path.
 * TEST INFRASTRUCTURE ONLY (see kvhp_oracle.h): never linked by product code.
 *
 * Build: oracle/Makefile -> oracle/liboracle.so (gcc -O2, no fast-math, so the
 * float/double evaluation order below is the one written).
 */
#include "kvhp_oracle.h"

#include <math.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* IEEE 754 binary16, written from the format definition: 1 sign bit, 5
 * exponent bits (bias 15), 10 fraction bits; subnormals scale 2^-24; results
 * rounded to nearest, ties to even.                                          */
uint16_t kvo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t mant = x & 0x7FFFFFu;
    if (exp == 0xFFu) {                       /* inf / nan */
        if (mant) return (uint16_t)(sign | 0x7E00u | (mant >> 13));
        return (uint16_t)(sign | 0x7C00u);
    }
    int e = (int)exp - 127 + 15;              /* re-biased exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {                             /* half subnormal or zero */
        if (e < -10) return (uint16_t)sign;
        mant |= 0x800000u;                    /* explicit leading one */
        int shift = 14 - e;                   /* value = mant * 2^-(shift+10) */
        uint32_t hm = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);         /* carry into exponent is exact */
    }
    uint32_t hm = mant >> 13;
    uint32_t rem = mant & 0x1FFFu;
    uint32_t h = sign | ((uint32_t)e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) h++;  /* may carry to inf */
    return (uint16_t)h;
}

float kvo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t mant = (uint32_t)h & 0x3FFu;
    uint32_t x;
    if (exp == 0) {
        if (mant == 0) {
            x = sign;
        } else {                              /* subnormal: mant * 2^-24 */
            float v = (float)mant * 5.9604644775390625e-8f;
            memcpy(&x, &v, sizeof x);
            x |= sign;
        }
    } else if (exp == 31) {
        x = sign | 0x7F800000u | (mant << 13);
    } else {
        x = sign | ((exp - 15 + 127) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &x, sizeof f);
    return f;
}

void kvo_f32_to_f16_array(const float* src, uint16_t* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = kvo_f32_to_f16(src[i]);
}

void kvo_f16_to_f32_array(const uint16_t* src, float* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = kvo_f16_to_f32(src[i]);
}

/* ------------------------------------------------------------------------ */
/* One causal attention row, reference src/cpu/ops.cpp:242-282:
 *   dot in double over D -> (float)dot * scale            (:249-253)
 *   running max initialised to -1e30f                     (:246)
 *   exp in float, sum of exps in double                   (:261-266)
 *   probabilities scaled by (float)(1/sum)                (:267-270)
 *   PV accumulated in double, stored as float             (:274-281)
 * `scores` is caller scratch of length >= nkeys. */
static void attend_row(const float* q_vec, const float* k_base,
                       const float* v_base, int64_t k_stride, int64_t nkeys,
                       int64_t D, float scale, float* scores, float* out_vec) {
    /* Four keys' dots (and below four output dims) are carried side by side
     * as independent chains; every element keeps its own operation order. */
    float max_score = -1e30f;
    int64_t j = 0;
    for (; j + 4 <= nkeys; j += 4) {
        const float* k0 = k_base + j * k_stride;
        const float* k1 = k0 + k_stride;
        const float* k2 = k1 + k_stride;
        const float* k3 = k2 + k_stride;
        double d0 = 0.0, d1 = 0.0, d2 = 0.0, d3 = 0.0;
        for (int64_t d = 0; d < D; ++d) {
            const double qd = (double)q_vec[d];
            d0 += qd * (double)k0[d];
            d1 += qd * (double)k1[d];
            d2 += qd * (double)k2[d];
            d3 += qd * (double)k3[d];
        }
        const double dots[4] = {d0, d1, d2, d3};
        for (int u = 0; u < 4; ++u) {
            float score = (float)dots[u] * scale;
            scores[j + u] = score;
            if (score > max_score) max_score = score;
        }
    }
    for (; j < nkeys; ++j) {
        const float* k_vec = k_base + j * k_stride;
        double dot = 0.0;
        for (int64_t d = 0; d < D; ++d) dot += (double)q_vec[d] * (double)k_vec[d];
        float score = (float)dot * scale;
        scores[j] = score;
        if (score > max_score) max_score = score;
    }
    double sum_exp = 0.0;
    for (j = 0; j < nkeys; ++j) {
        float e = expf(scores[j] - max_score);
        scores[j] = e;
        sum_exp += (double)e;
    }
    float inv_sum = (float)(1.0 / sum_exp);
    for (j = 0; j < nkeys; ++j) scores[j] *= inv_sum;
    int64_t d = 0;
    for (; d + 4 <= D; d += 4) {
        double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
        for (j = 0; j < nkeys; ++j) {
            const double p = (double)scores[j];
            const float* vr = v_base + j * k_stride + d;
            a0 += p * (double)vr[0];
            a1 += p * (double)vr[1];
            a2 += p * (double)vr[2];
            a3 += p * (double)vr[3];
        }
        out_vec[d] = (float)a0;
        out_vec[d + 1] = (float)a1;
        out_vec[d + 2] = (float)a2;
        out_vec[d + 3] = (float)a3;
    }
    for (; d < D; ++d) {
        double acc = 0.0;
        for (j = 0; j < nkeys; ++j)
            acc += (double)scores[j] * (double)v_base[j * k_stride + d];
        out_vec[d] = (float)acc;
    }
}

void kvo_causal_gqa_rows(const float* q, const float* k, const float* v,
                         float* out, int64_t S, int64_t Hq, int64_t Hkv,
                         int64_t D, int64_t row_begin, int64_t row_end,
                         int nthreads) {
    if (row_begin < 0) row_begin = 0;
    if (row_end > S) row_end = S;
    if (row_end <= row_begin) return;
    int64_t group = Hq / Hkv;                               /* :232 */
    float scale = 1.0f / sqrtf((float)D);                   /* :234 */
    int64_t nrows = row_end - row_begin;
    int64_t total = Hq * nrows;
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel num_threads(nthreads) if (nthreads > 1)
    {
        float* scores = (float*)malloc(sizeof(float) * (size_t)(row_end > 0 ? row_end : 1));
#pragma omp for schedule(dynamic, 4)
        for (int64_t w = 0; w < total; ++w) {
            int64_t qh = w / nrows;
            int64_t i = row_begin + (w % nrows);
            int64_t kvh = qh / group;                       /* :240 */
            attend_row(q + (i * Hq + qh) * D, k + kvh * D, v + kvh * D,
                       Hkv * D, i + 1, D, scale, scores,
                       out + (i * Hq + qh) * D);
        }
        free(scores);
    }
}

/* The rows listed in rows[0..nrows) (each in [0, S)), written to
 * out[nrows][Hq][D]: the same attend_row arithmetic as kvo_causal_gqa_rows,
 * for checking scattered rows of long prompts without a full-size output. */
void kvo_causal_gqa_rowlist(const float* q, const float* k, const float* v,
                            float* out, int64_t S, int64_t Hq, int64_t Hkv,
                            int64_t D, const int64_t* rows, int64_t nrows,
                            int nthreads) {
    if (nrows <= 0) return;
    int64_t group = Hq / Hkv;                               /* :232 */
    float scale = 1.0f / sqrtf((float)D);                   /* :234 */
    int64_t total = Hq * nrows;
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel num_threads(nthreads) if (nthreads > 1)
    {
        float* scores = (float*)malloc(sizeof(float) * (size_t)(S > 0 ? S : 1));
#pragma omp for schedule(dynamic, 4)
        for (int64_t w = 0; w < total; ++w) {
            int64_t qh = w % Hq;
            int64_t j = w / Hq;
            int64_t i = rows[j];
            if (i < 0 || i >= S) continue;
            int64_t kvh = qh / group;                       /* :240 */
            attend_row(q + (i * Hq + qh) * D, k + kvh * D, v + kvh * D,
                       Hkv * D, i + 1, D, scale, scores,
                       out + (j * Hq + qh) * D);
        }
        free(scores);
    }
}

void kvo_causal_gqa(const float* q, const float* k, const float* v, float* out,
                    int64_t S, int64_t Hq, int64_t Hkv, int64_t D) {
    kvo_causal_gqa_rows(q, k, v, out, S, Hq, Hkv, D, 0, S, 1);
}

void kvo_decode_attention(const float* q, const float* k, const float* v,
                          const int32_t* seq_lens, float* out, int64_t B,
                          int64_t Hq, int64_t Hkv, int64_t D, int64_t cap,
                          int nthreads) {
    int64_t group = Hq / Hkv;
    float scale = 1.0f / sqrtf((float)D);
    int64_t total = B * Hq;
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel num_threads(nthreads) if (nthreads > 1)
    {
        float* scores = (float*)malloc(sizeof(float) * (size_t)(cap > 0 ? cap : 1));
#pragma omp for schedule(dynamic, 1)
        for (int64_t w = 0; w < total; ++w) {
            int64_t b = w / Hq, qh = w % Hq, kvh = qh / group;
            int64_t L = seq_lens[b];
            float* o = out + (b * Hq + qh) * D;
            if (L <= 0) {
                for (int64_t d = 0; d < D; ++d) o[d] = 0.0f;
                continue;
            }
            if (L > cap) L = cap;
            const float* kh = k + (b * Hkv + kvh) * cap * D;
            const float* vh = v + (b * Hkv + kvh) * cap * D;
            attend_row(q + (b * Hq + qh) * D, kh, vh, D, L, D, scale, scores, o);
        }
        free(scores);
    }
}

/* ------------------------------------------------------------------------ */
/* Split-K decode.  The reference describes but never implements it
 * (docs/reports/P7.md:13,32-34; scratch sized (D+2) floats per split at
 * src/model/forward_gpu.cu:100).  Scores follow ops.cpp:249-253; each split
 * keeps its own max, so exp arguments are relative to the split max. */
void kvo_decode_split_partial(const float* q_vec, const float* k_head,
                              const float* v_head, int64_t D, int64_t t0,
                              int64_t t1, float* m_out, double* l_out,
                              double* o) {
    float scale = 1.0f / sqrtf((float)D);
    for (int64_t d = 0; d < D; ++d) o[d] = 0.0;
    if (t1 <= t0) {
        *m_out = -INFINITY;
        *l_out = 0.0;
        return;
    }
    float m = -INFINITY;
    float* scores = (float*)malloc(sizeof(float) * (size_t)(t1 - t0));
    for (int64_t t = t0; t < t1; ++t) {
        const float* kv = k_head + t * D;
        double dot = 0.0;
        for (int64_t d = 0; d < D; ++d) dot += (double)q_vec[d] * (double)kv[d];
        float s = (float)dot * scale;
        scores[t - t0] = s;
        if (s > m) m = s;
    }
    double l = 0.0;
    for (int64_t t = t0; t < t1; ++t) {
        float p = expf(scores[t - t0] - m);
        l += (double)p;
        const float* vv = v_head + t * D;
        for (int64_t d = 0; d < D; ++d) o[d] += (double)p * (double)vv[d];
    }
    free(scores);
    *m_out = m;
    *l_out = l;
}

/* M = max_j m_j;  Lsum = sum_j l_j e^(m_j-M);  out = sum_j o_j e^(m_j-M) / Lsum.
 * Empty partials (m=-inf, l=0) carry weight 0. */
void kvo_lse_merge(const float* m, const double* l, const double* o,
                   int64_t n, int64_t D, float* out) {
    double M = -INFINITY;
    for (int64_t j = 0; j < n; ++j)
        if (l[j] > 0.0 && (double)m[j] > M) M = (double)m[j];
    if (M == -INFINITY) {
        for (int64_t d = 0; d < D; ++d) out[d] = 0.0f;
        return;
    }
    double lsum = 0.0;
    for (int64_t j = 0; j < n; ++j)
        if (l[j] > 0.0) lsum += l[j] * exp((double)m[j] - M);
    for (int64_t d = 0; d < D; ++d) {
        double acc = 0.0;
        for (int64_t j = 0; j < n; ++j)
            if (l[j] > 0.0) acc += o[j * D + d] * exp((double)m[j] - M);
        out[d] = (float)(acc / lsum);
    }
}

void kvo_decode_attention_splitk(const float* q, const float* k,
                                 const float* v, const int32_t* seq_lens,
                                 float* out, int64_t B, int64_t Hq,
                                 int64_t Hkv, int64_t D, int64_t cap,
                                 int64_t chunk, int nthreads) {
    int64_t group = Hq / Hkv;
    if (chunk < 1) chunk = 1;
    int64_t total = B * Hq;
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1) if (nthreads > 1)
    for (int64_t w = 0; w < total; ++w) {
        int64_t b = w / Hq, qh = w % Hq, kvh = qh / group;
        int64_t L = seq_lens[b];
        if (L > cap) L = cap;
        float* o_out = out + (b * Hq + qh) * D;
        if (L <= 0) {
            for (int64_t d = 0; d < D; ++d) o_out[d] = 0.0f;
            continue;
        }
        int64_t n = (L + chunk - 1) / chunk;
        float* ms = (float*)malloc(sizeof(float) * (size_t)n);
        double* ls = (double*)malloc(sizeof(double) * (size_t)n);
        double* os = (double*)malloc(sizeof(double) * (size_t)(n * D));
        const float* kh = k + (b * Hkv + kvh) * cap * D;
        const float* vh = v + (b * Hkv + kvh) * cap * D;
        for (int64_t j = 0; j < n; ++j) {
            int64_t t0 = j * chunk, t1 = t0 + chunk < L ? t0 + chunk : L;
            kvo_decode_split_partial(q + (b * Hq + qh) * D, kh, vh, D, t0, t1,
                                     &ms[j], &ls[j], &os[j * D]);
        }
        kvo_lse_merge(ms, ls, os, n, D, o_out);
        free(ms);
        free(ls);
        free(os);
    }
}

/* ------------------------------------------------------------------------ */
/* Contiguous append, reference runtime/kv_cache.cu:20-35:
 *   src offset (t*Hkv + h)*D + d  ->  dst offset (h*max_seq + pos)*D + d,
 *   pos = start_pos + t, skipped when pos >= max_seq (:26). */
void kvo_append_kv(const uint16_t* src_k, const uint16_t* src_v,
                   uint16_t* dst_k, uint16_t* dst_v, int64_t num_tokens,
                   int64_t start_pos, int64_t Hkv, int64_t max_seq, int64_t D) {
    for (int64_t t = 0; t < num_tokens; ++t) {
        int64_t pos = start_pos + t;
        if (pos >= max_seq || pos < 0) continue;
        for (int64_t h = 0; h < Hkv; ++h) {
            memcpy(dst_k + (h * max_seq + pos) * D, src_k + (t * Hkv + h) * D,
                   (size_t)D * 2);
            memcpy(dst_v + (h * max_seq + pos) * D, src_v + (t * Hkv + h) * D,
                   (size_t)D * 2);
        }
    }
}

/* Paged form of the same map: dst = pool[h][bt[b][pos/page]][pos%page][:].
 * With an identity table this is byte-identical to kvo_append_kv with
 * max_seq = max_pages*page (layout comment runtime/kv_cache.h:9-11). */
void kvo_paged_append(const uint16_t* src_k, const uint16_t* src_v,
                      uint16_t* pool_k, uint16_t* pool_v,
                      const int32_t* block_tables, int64_t max_pages,
                      const int32_t* start_pos, int64_t B, int64_t T,
                      int64_t Hkv, int64_t D, int64_t P, int64_t page) {
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t t = 0; t < T; ++t) {
            int64_t pos = (int64_t)start_pos[b] + t;
            if (pos < 0) continue;
            int64_t pi = pos / page;
            if (pi >= max_pages) continue;
            int64_t pid = block_tables[b * max_pages + pi];
            if (pid < 0 || pid >= P) continue;
            for (int64_t h = 0; h < Hkv; ++h) {
                int64_t src = ((b * T + t) * Hkv + h) * D;
                int64_t dst = ((h * P + pid) * page + pos % page) * D;
                memcpy(pool_k + dst, src_k + src, (size_t)D * 2);
                memcpy(pool_v + dst, src_v + src, (size_t)D * 2);
            }
        }
    }
}

void kvo_paged_gather(const uint16_t* pool_k, const uint16_t* pool_v,
                      const int32_t* block_tables, int64_t max_pages,
                      const int32_t* seq_lens, int64_t B, int64_t Hkv,
                      int64_t D, int64_t P, int64_t page, int64_t max_len,
                      uint16_t* out_k, uint16_t* out_v) {
    for (int64_t b = 0; b < B; ++b) {
        int64_t L = seq_lens[b];
        for (int64_t h = 0; h < Hkv; ++h) {
            for (int64_t s = 0; s < max_len; ++s) {
                int64_t o = ((b * Hkv + h) * max_len + s) * D;
                int64_t pi = s / page;
                int64_t pid = (s < L && pi < max_pages) ? block_tables[b * max_pages + pi] : -1;
                if (pid < 0 || pid >= P) {
                    memset(out_k + o, 0, (size_t)D * 2);
                    memset(out_v + o, 0, (size_t)D * 2);
                    continue;
                }
                int64_t src = ((h * P + pid) * page + s % page) * D;
                memcpy(out_k + o, pool_k + src, (size_t)D * 2);
                memcpy(out_v + o, pool_v + src, (size_t)D * 2);
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* RMSNorm, reference ops.cpp:26-51: sum of squares in double, rsqrt in
 * double cast to float, out = x * r * w in float. */
void kvo_rmsnorm(const float* x, const float* w, float* out, int64_t rows,
                 int64_t dim, float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * dim;
        float* orow = out + r * dim;
        double ss = 0.0;
        for (int64_t c = 0; c < dim; ++c) {
            double t = (double)xr[c];
            ss += t * t;
        }
        double mean = ss / (double)dim;
        float rs = (float)(1.0 / sqrt(mean + (double)eps));
        for (int64_t c = 0; c < dim; ++c) orow[c] = xr[c] * rs * w[c];
    }
}

/* C[M][N] = A[M][K] * B[N][K]^T, reference matmul_transB_blocked
 * (ops.cpp:76-114): 64-wide K blocks, each block's dot in double (products
 * of the floats widened to double, added in k order), converted to float and
 * added to the float output in block order. */
static void matmul_scalar(const float* A, const float* B, float* C, int64_t M,
                          int64_t K, int64_t N, int nthreads) {
#pragma omp parallel for num_threads(nthreads) schedule(static) if (nthreads > 1)
    for (int64_t n = 0; n < N; ++n) {
        const float* brow = B + n * K;
        for (int64_t m = 0; m < M; ++m) {
            const float* arow = A + m * K;
            float c = 0.0f;
            for (int64_t k0 = 0; k0 < K; k0 += 64) {
                int64_t k1 = k0 + 64 < K ? k0 + 64 : K;
                double s = 0.0;
                for (int64_t k = k0; k < k1; ++k) s += (double)arow[k] * (double)brow[k];
                c += (float)s;
            }
            C[m * N + n] = c;
        }
    }
}

#if defined(__x86_64__)
#include <immintrin.h>

/* The same arithmetic, 4 rows x 8 columns at a time in AVX2 registers: lane j
 * of a vector is one output element, so every element still sees exactly the
 * scalar sequence (a separate IEEE double multiply and add per k in k order,
 * no FMA: the target enables AVX2 only; round-to-nearest float conversion
 * and float add per 64-block).  A rows of the tile beyond M repeat row M-1
 * and are not stored.  ad: A rows [mb][K] already widened to double; bp: the
 * panel's columns [K][8] widened, zero past N. */
__attribute__((target("avx2")))
static void mm_tile_rows_avx2(const double* ad, int64_t mb, const double* bp, int64_t K,
                              float* C, int64_t ldc, int64_t nw) {
    for (int64_t m0 = 0; m0 < mb; m0 += 4) {
        const double* r0 = ad + m0 * K;
        const double* r1 = ad + (m0 + 1 < mb ? m0 + 1 : mb - 1) * K;
        const double* r2 = ad + (m0 + 2 < mb ? m0 + 2 : mb - 1) * K;
        const double* r3 = ad + (m0 + 3 < mb ? m0 + 3 : mb - 1) * K;
        __m128 c[4][2];
        for (int i = 0; i < 4; ++i) c[i][0] = c[i][1] = _mm_setzero_ps();
        for (int64_t k0 = 0; k0 < K; k0 += 64) {
            const int64_t k1 = k0 + 64 < K ? k0 + 64 : K;
            __m256d s00 = _mm256_setzero_pd(), s01 = _mm256_setzero_pd();
            __m256d s10 = _mm256_setzero_pd(), s11 = _mm256_setzero_pd();
            __m256d s20 = _mm256_setzero_pd(), s21 = _mm256_setzero_pd();
            __m256d s30 = _mm256_setzero_pd(), s31 = _mm256_setzero_pd();
            for (int64_t k = k0; k < k1; ++k) {
                const __m256d b0 = _mm256_load_pd(bp + k * 8);
                const __m256d b1 = _mm256_load_pd(bp + k * 8 + 4);
                __m256d a = _mm256_broadcast_sd(r0 + k);
                s00 = _mm256_add_pd(s00, _mm256_mul_pd(a, b0));
                s01 = _mm256_add_pd(s01, _mm256_mul_pd(a, b1));
                a = _mm256_broadcast_sd(r1 + k);
                s10 = _mm256_add_pd(s10, _mm256_mul_pd(a, b0));
                s11 = _mm256_add_pd(s11, _mm256_mul_pd(a, b1));
                a = _mm256_broadcast_sd(r2 + k);
                s20 = _mm256_add_pd(s20, _mm256_mul_pd(a, b0));
                s21 = _mm256_add_pd(s21, _mm256_mul_pd(a, b1));
                a = _mm256_broadcast_sd(r3 + k);
                s30 = _mm256_add_pd(s30, _mm256_mul_pd(a, b0));
                s31 = _mm256_add_pd(s31, _mm256_mul_pd(a, b1));
            }
            c[0][0] = _mm_add_ps(c[0][0], _mm256_cvtpd_ps(s00));
            c[0][1] = _mm_add_ps(c[0][1], _mm256_cvtpd_ps(s01));
            c[1][0] = _mm_add_ps(c[1][0], _mm256_cvtpd_ps(s10));
            c[1][1] = _mm_add_ps(c[1][1], _mm256_cvtpd_ps(s11));
            c[2][0] = _mm_add_ps(c[2][0], _mm256_cvtpd_ps(s20));
            c[2][1] = _mm_add_ps(c[2][1], _mm256_cvtpd_ps(s21));
            c[3][0] = _mm_add_ps(c[3][0], _mm256_cvtpd_ps(s30));
            c[3][1] = _mm_add_ps(c[3][1], _mm256_cvtpd_ps(s31));
        }
        for (int i = 0; i < 4 && m0 + i < mb; ++i) {
            float row[8];
            _mm_storeu_ps(row, c[i][0]);
            _mm_storeu_ps(row + 4, c[i][1]);
            for (int64_t j = 0; j < nw; ++j) C[(m0 + i) * ldc + j] = row[j];
        }
    }
}

/* Rows in blocks of 256 (widened once, shared by the threads), columns in
 * panels of 8 (one per task, widened into the task's buffer). */
static int matmul_avx2(const float* A, const float* B, float* C, int64_t M, int64_t K,
                       int64_t N, int nthreads) {
    const int64_t MB = 256;
    double* ad = (double*)aligned_alloc(64, sizeof(double) * (size_t)(MB * K + 8));
    if (!ad) return -1;
    const int64_t panels = (N + 7) / 8;
    int failed = 0;
    for (int64_t m0 = 0; m0 < M && !failed; m0 += MB) {
        const int64_t mb = M - m0 < MB ? M - m0 : MB;
#pragma omp parallel for num_threads(nthreads) schedule(static) if (nthreads > 1)
        for (int64_t i = 0; i < mb * K; ++i) ad[i] = (double)A[m0 * K + i];
#pragma omp parallel num_threads(nthreads) if (nthreads > 1)
        {
            double* bp = (double*)aligned_alloc(64, sizeof(double) * (size_t)(K * 8 + 8));
            if (!bp) {
#pragma omp atomic write
                failed = 1;
            }
#pragma omp for schedule(dynamic, 4)
            for (int64_t p = 0; p < panels; ++p) {
                if (!bp) continue;
                const int64_t n0 = p * 8;
                const int64_t nw = N - n0 < 8 ? N - n0 : 8;
                for (int64_t j = 0; j < 8; ++j) {
                    const float* brow = B + (n0 + (j < nw ? j : 0)) * K;
                    for (int64_t k = 0; k < K; ++k) bp[k * 8 + j] = j < nw ? (double)brow[k] : 0.0;
                }
                mm_tile_rows_avx2(ad, mb, bp, K, C + m0 * N + n0, N, nw);
            }
            free(bp);
        }
    }
    free(ad);
    return failed ? -1 : 0;
}
#endif

void kvo_matmul_transB(const float* A, const float* B, float* C, int64_t M,
                       int64_t K, int64_t N, int nthreads) {
    if (nthreads < 1) nthreads = 1;
#if defined(__x86_64__)
    if (M >= 4 && __builtin_cpu_supports("avx2") && matmul_avx2(A, B, C, M, K, N, nthreads) == 0)
        return;
#endif
    matmul_scalar(A, B, C, M, K, N, nthreads);
}

/* The scalar form alone (the vector form is checked against it). */
void kvo_matmul_transB_scalar(const float* A, const float* B, float* C, int64_t M,
                              int64_t K, int64_t N, int nthreads) {
    matmul_scalar(A, B, C, M, K, N, nthreads < 1 ? 1 : nthreads);
}

/* Half-split RoPE, reference ops.cpp:165-221: inv_freq in float via powf,
 * angle = (float)pos * inv_freq, cosf/sinf, x1*c - x2*s and x2*c + x1*s. */
void kvo_apply_rope(float* q, float* k, int64_t S, int64_t Hq, int64_t Hkv,
                    int64_t D, int64_t start_pos, float theta) {
    int64_t half = D / 2;
    float* inv = (float*)malloc(sizeof(float) * (size_t)half);
    float* cb = (float*)malloc(sizeof(float) * (size_t)half);
    float* sb = (float*)malloc(sizeof(float) * (size_t)half);
    for (int64_t i = 0; i < half; ++i)
        inv[i] = 1.0f / powf(theta, (float)(2 * i) / (float)D);
    for (int64_t s = 0; s < S; ++s) {
        int64_t pos = start_pos + s;
        for (int64_t i = 0; i < half; ++i) {
            float a = (float)pos * inv[i];
            cb[i] = cosf(a);
            sb[i] = sinf(a);
        }
        for (int pass = 0; pass < 2; ++pass) {
            float* base = pass == 0 ? q : k;
            int64_t H = pass == 0 ? Hq : Hkv;
            if (!base) continue;
            for (int64_t h = 0; h < H; ++h) {
                float* vec = base + (s * H + h) * D;
                for (int64_t i = 0; i < half; ++i) {
                    float x1 = vec[i], x2 = vec[half + i];
                    vec[i] = x1 * cb[i] - x2 * sb[i];
                    vec[half + i] = x2 * cb[i] + x1 * sb[i];
                }
            }
        }
    }
    free(inv);
    free(cb);
    free(sb);
}

/* SwiGLU, reference ops.cpp:286-297: silu(g) = g / (1 + expf(-g)). */
void kvo_swiglu(const float* gate, const float* up, float* out, int64_t count) {
    for (int64_t i = 0; i < count; ++i) {
        float g = gate[i];
        float s = g / (1.0f + expf(-g));
        out[i] = s * up[i];
    }
}
