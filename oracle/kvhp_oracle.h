/*
 * kvhp_oracle.h -- CPU restatement of the serving-engine KV-cache hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * kernels in serving-engine_amd/csrc.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it.  No product code path links it,
 * and nothing here is ever used as a fallback for the GPU path.
 *
 * Every function names the reference source (path:line under the reference
 * tree) whose arithmetic it restates.  Tensors are row-major.  Attention
 * inputs are float arrays that hold fp16-rounded values, as the reference
 * tests pass them (tests/test_attention.cpp:75-77); KV movement works on raw
 * 16-bit patterns so "bit-exact" is literal.
 *
 * Pinning (how each function is checked, see tests/test_oracle.py):
 *   kvo_causal_gqa       bit-exact vs the reference src/cpu/ops.cpp compiled
 *                        under oracle/_ref, golden fixtures, KAT row0 == v[0]
 *   kvo_decode_attention == last row of kvo_causal_gqa (invariant), KATs
 *                        L=1 -> V[0], equal keys -> mean(V), dominant key
 *   kvo_decode_split_*   split-count invariance, single split == identity,
 *   kvo_lse_merge        brute force over all split points on tiny L
 *   kvo_append_kv        closed-form index map of runtime/kv_cache.cu:29-32
 *   kvo_paged_*          identity block table == contiguous layout,
 *                        random permutations, drop rules
 *   kvo_rmsnorm/rope/    bit-exact vs oracle/_ref and the reference KATs
 *   swiglu/matmul        (tests/test_cpu_ops.cpp:12-110); the vectorised
 *                        matmul also bit for bit vs its scalar form
 *   kvo_f32_to_f16       against numpy float16 (IEEE RNE) on all boundaries
 */
#ifndef KVHP_ORACLE_H
#define KVHP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- IEEE binary16 <-> binary32 (round to nearest even) ---------------- */
uint16_t kvo_f32_to_f16(float x);
float kvo_f16_to_f32(uint16_t h);
void kvo_f32_to_f16_array(const float* src, uint16_t* dst, int64_t n);
void kvo_f16_to_f32_array(const uint16_t* src, float* dst, int64_t n);

/* ---- Attention (ops.cpp:223-284) ---------------------------------------- */
/* q [S][Hq][D], k/v [S][Hkv][D], out [S][Hq][D].  Rows are independent, so
 * kvo_causal_gqa_rows computes only rows [row_begin,row_end) with identical
 * per-row arithmetic (used to sample rows of long prompts).  nthreads>1 splits
 * the (q_head,row) loop across OpenMP threads without changing any row's
 * arithmetic. */
void kvo_causal_gqa(const float* q, const float* k, const float* v, float* out,
                    int64_t S, int64_t Hq, int64_t Hkv, int64_t D);
void kvo_causal_gqa_rows(const float* q, const float* k, const float* v,
                         float* out, int64_t S, int64_t Hq, int64_t Hkv,
                         int64_t D, int64_t row_begin, int64_t row_end,
                         int nthreads);
/* Rows rows[0..nrows) only (any order, each in [0,S)), output
 * out[nrows][Hq][D]; per-row arithmetic identical to kvo_causal_gqa. */
void kvo_causal_gqa_rowlist(const float* q, const float* k, const float* v,
                            float* out, int64_t S, int64_t Hq, int64_t Hkv,
                            int64_t D, const int64_t* rows, int64_t nrows,
                            int nthreads);

/* Decode: one query per sequence over its first seq_lens[b] cached keys.
 * q [B][Hq][D]; k/v contiguous [B][Hkv][cap][D]; out [B][Hq][D].
 * Arithmetic is that of the last causal row (ops.cpp:242-282).  A sequence
 * with seq_len <= 0 produces zeros. */
void kvo_decode_attention(const float* q, const float* k, const float* v,
                          const int32_t* seq_lens, float* out, int64_t B,
                          int64_t Hq, int64_t Hkv, int64_t D, int64_t cap,
                          int nthreads);

/* Split-K decode for one (q vector, kv head): partial over tokens [t0,t1):
 * m = max score, l = sum exp(s-m), o[d] = sum exp(s-m) v[d] (unnormalised).
 * Empty range -> m=-inf, l=0, o=0. */
void kvo_decode_split_partial(const float* q_vec, const float* k_head,
                              const float* v_head, int64_t D, int64_t t0,
                              int64_t t1, float* m, double* l, double* o);
/* Log-sum-exp merge of n partials (m[n], l[n], o[n][D]) -> out[D].
 * All-empty -> zeros. */
void kvo_lse_merge(const float* m, const double* l, const double* o,
                   int64_t n, int64_t D, float* out);
/* Full split-K decode (partials over `num_splits` equal page-aligned chunks,
 * then merge) -- the restated algorithm the GPU kernel implements. */
void kvo_decode_attention_splitk(const float* q, const float* k,
                                 const float* v, const int32_t* seq_lens,
                                 float* out, int64_t B, int64_t Hq,
                                 int64_t Hkv, int64_t D, int64_t cap,
                                 int64_t chunk, int nthreads);

/* ---- KV movement (runtime/kv_cache.cu:8-36) ------------------------------ */
/* src [T][Hkv][D] -> dst [Hkv][max_seq][D] at start_pos..; pos>=max_seq dropped. */
void kvo_append_kv(const uint16_t* src_k, const uint16_t* src_v,
                   uint16_t* dst_k, uint16_t* dst_v, int64_t num_tokens,
                   int64_t start_pos, int64_t Hkv, int64_t max_seq, int64_t D);
/* Paged pool [Hkv][P][page][D]; block table [B][max_pages]; token pos of
 * (b,t) = start_pos[b]+t.  Dropped: pos<0, pos/page>=max_pages, page id
 * outside [0,P). */
void kvo_paged_append(const uint16_t* src_k, const uint16_t* src_v,
                      uint16_t* pool_k, uint16_t* pool_v,
                      const int32_t* block_tables, int64_t max_pages,
                      const int32_t* start_pos, int64_t B, int64_t T,
                      int64_t Hkv, int64_t D, int64_t P, int64_t page);
/* out [B][Hkv][max_len][D]; positions >= seq_lens[b] (or invalid ids) = 0. */
void kvo_paged_gather(const uint16_t* pool_k, const uint16_t* pool_v,
                      const int32_t* block_tables, int64_t max_pages,
                      const int32_t* seq_lens, int64_t B, int64_t Hkv,
                      int64_t D, int64_t P, int64_t page, int64_t max_len,
                      uint16_t* out_k, uint16_t* out_v);

/* ---- Supporting ops for the full-model decode (ops.cpp) ----------------- */
void kvo_rmsnorm(const float* x, const float* w, float* out, int64_t rows,
                 int64_t dim, float eps);                       /* :26-51  */
void kvo_matmul_transB(const float* A, const float* B, float* C, int64_t M,
                       int64_t K, int64_t N, int nthreads);
/* The scalar form of kvo_matmul_transB alone (kvo_matmul_transB uses AVX2
 * registers where the CPU has them, with the same per-element arithmetic;
 * tests check the two bit for bit). */
void kvo_matmul_transB_scalar(const float* A, const float* B, float* C, int64_t M,
                              int64_t K, int64_t N, int nthreads);     /* :76-114 */
void kvo_apply_rope(float* q, float* k, int64_t S, int64_t Hq, int64_t Hkv,
                    int64_t D, int64_t start_pos, float theta); /* :165-221 */
void kvo_swiglu(const float* gate, const float* up, float* out,
                int64_t count);                                 /* :286-297 */

#ifdef __cplusplus
}
#endif
#endif
