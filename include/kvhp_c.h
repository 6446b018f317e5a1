/*
 * kvhp_c.h -- C ABI of the MI355X (gfx950) KV-cache hot path.
 *
 * This is the drop-in boundary for the serving-engine KV-cache/attention
 * path.  Each entry point names the reference interface it replaces
 * (path:line in the reference tree).  The C++ mirror of the reference API
 * (engine::KVCache, engine::cuda::append_kv_cache, decode_gqa_split, ...)
 * lives in serving-engine_amd/engine/ and calls only these functions.
 *
 * Conventions (kept from the reference, src/cuda/kernels.h and
 * src/runtime/kv_cache.h):
 *   - every tensor argument is a raw device pointer the caller owns;
 *     fp16 tensors are IEEE binary16 (passed as void*), indices int32;
 *   - work is enqueued on `stream` (a hipStream_t; NULL = default stream)
 *     and never synchronised;
 *   - empty work (zero tokens / zero length) is a no-op returning KVHP_OK.
 * Differences:
 *   - errors are returned as a status code (< 0) instead of a C++ throw; the
 *     message is available from kvhp_last_error() (thread-local).  The C++
 *     mirror turns a non-zero status into std::runtime_error as the
 *     reference's CUDA_CHECK did (src/common/cuda_utils.h:12-21).
 *   - decode with seq_len <= 0 writes zeros (the reference leaves the output
 *     untouched, src/cuda/decode_attention_split.cu:45-46).
 */
#ifndef KVHP_C_H
#define KVHP_C_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVHP_OK 0
#define KVHP_ERR_INVALID (-1)     /* bad shape / pointer / stride argument  */
#define KVHP_ERR_UNSUPPORTED (-2) /* valid but not implemented (e.g. D>256) */
#define KVHP_ERR_WORKSPACE (-3)   /* caller workspace too small             */
#define KVHP_ERR_HIP (-4)         /* HIP runtime error (launch / alloc)     */

#define KVHP_PAGE_SIZE 16         /* tokens per KV page                      */

/* Strided or paged view of one K or V cache, the reference KVView
 * (src/cuda/kv_view.h:17-31) extended with the block table its comment
 * plans for (kv_view.h:9-10).
 *   block_table == NULL (strided):
 *     elem(b,h,s,d) = data[b*stride_b + h*stride_h + s*stride_s + d*stride_d]
 *   block_table != NULL (paged; pool laid out [Hkv][num_pages][16][D]):
 *     elem(b,h,s,d) = data[h*stride_h
 *                         + (block_table[b*max_pages + s/16]*16 + s%16)*stride_s
 *                         + d*stride_d]
 *   Attention kernels require stride_d == 1 and 16-byte aligned rows. */
typedef struct kvhp_kv_view {
    const void* data;
    int64_t stride_b;
    int64_t stride_h;
    int64_t stride_s;
    int64_t stride_d;
    const int32_t* block_table;
    int32_t max_pages;   /* block-table row length (pages per sequence)       */
    int32_t page_size;   /* must be KVHP_PAGE_SIZE in paged mode              */
    int32_t num_pages;   /* pool capacity; page ids are clamped into range   */
    int32_t reserved;
} kvhp_kv_view;

/* Message of the last failing call on this thread ("" if none). */
const char* kvhp_last_error(void);
/* ABI version of this library (KVHP_ABI_VERSION). */
int kvhp_abi_version(void);
#define KVHP_ABI_VERSION 1
/* Build id of this library: the first 16 hex digits of the SHA-256 of its
 * sources (the .hip, then the .h files of its csrc directory, each set in
 * name order, then this header),
 * fixed when the library is linked, so a result can be tied to the sources
 * it ran. */
const char* kvhp_build_id(void);

/* Streaming-read calibration, the reference's read-bandwidth probe
 * (src/cuda/read_bandwidth.cu:8-118; its measured ceiling is the roofline of
 * docs/GATES.md:21): reads `bytes` (rounded down to 16) of device memory
 * once with 16-byte non-temporal loads and writes nothing (sink, 4 bytes of
 * device memory, is written only if the data fold equals a fixed constant).
 * Time it over a buffer larger than the 256 MB MALL with the caches flushed
 * to get the device's achievable read bandwidth. */
int kvhp_stream_read(const void* buf, size_t bytes, void* sink, void* stream);

/* Paged-read calibration beside the streaming probe above (the same
 * reference probe, src/cuda/read_bandwidth.cu:8-118, for the access pattern
 * of a paged decode): reads the pages page_ids[0..n_ids) of `pool`
 * (pool_bytes of device memory cut into pages of page_bytes = 2048 or 4096,
 * the page of one KV head at D = 64 or 128, or 8192 / 16384 / 32768 to
 * measure coarser layouts) once each with 16-byte
 * non-temporal loads; ids outside the pool are clamped into it.  Writes
 * nothing but possibly the 4-byte sink, as above.  With a random page order
 * and as many pages as a decode step reads, its rate is the ceiling of that
 * step's page reads. */
int kvhp_page_read(const void* pool, int64_t pool_bytes, const int32_t* page_ids, int64_t n_ids,
                   int page_bytes, void* sink, void* stream);

/* Replaces engine::cuda::append_kv_cache (src/runtime/kv_cache.h:80-91,
 * kernel src/runtime/kv_cache.cu:8-61).  src [num_tokens][Hkv][D] token-major
 * -> dst head base [Hkv][max_seq][D] at positions start_pos.., positions
 * >= max_seq dropped.  Bit-exact copy. */
int kvhp_append_kv(const void* src_k, const void* src_v, void* dst_k_head_base,
                   void* dst_v_head_base, int num_tokens, int start_pos,
                   int num_kv_heads, int max_seq, int head_dim, void* stream);

/* Paged form of append_kv_cache (paging planned at src/cuda/kv_view.h:9-10,
 * never built in the reference).  src [batch][num_tokens][Hkv][D]; token
 * (b,t) goes to position start_pos[b]+t (start_pos: device int32[batch]) of
 * pool [Hkv][num_pages][16][D] through block_tables [batch][max_pages].
 * Dropped: pos < 0, pos/16 >= max_pages, page id outside [0,num_pages). */
int kvhp_paged_append_kv(const void* src_k, const void* src_v, void* pool_k,
                         void* pool_v, const int32_t* block_tables,
                         int max_pages, const int32_t* start_pos, int batch,
                         int num_tokens, int num_kv_heads, int head_dim,
                         int num_pages, void* stream);

/* Paged gather (the address map of KVView::get_ptr, src/cuda/kv_view.h:24-30,
 * made explicit): out [batch][Hkv][max_len][D] <- pool through the block
 * table for s < seq_lens[b]; other positions are written as zero. */
int kvhp_paged_gather_kv(const void* pool_k, const void* pool_v,
                         const int32_t* block_tables, int max_pages,
                         const int32_t* seq_lens, int batch, int num_kv_heads,
                         int head_dim, int num_pages, int max_len, void* out_k,
                         void* out_v, void* stream);

/* Split slots per sequence the decode entry points use when num_splits == 0
 * (the workspace holds this many partials per (sequence, query head)).  For
 * 8 or more sequences the auto mode cuts each sequence into its own number
 * of splits, at most this many, chosen on the device from the lengths so
 * that the batch fills the GPU's resident waves about once. */
int kvhp_decode_auto_splits(int batch, int num_kv_heads, int head_dim,
                            int max_seq_len);
/* Bytes of workspace kvhp_decode_attention needs for these arguments
 * (num_splits == 0 -> auto): fp32 split partials (o[D], m, l) per
 * (sequence, query head, split); 0 when one split covers max_seq_len. */
size_t kvhp_decode_workspace_bytes(int batch, int num_q_heads,
                                   int num_kv_heads, int head_dim,
                                   int max_seq_len, int num_splits);
/* Zero a caller workspace (enqueued on stream).  Optional: the decode entry
 * points never read workspace bytes they did not write in the same call. */
int kvhp_decode_workspace_init(void* workspace, size_t workspace_bytes,
                               void* stream);

/* Replaces engine::cuda::decode_gqa_split (src/cuda/kernels.h:117-133,
 * src/cuda/decode_attention_split.cu:183-214), with the split-K partials and
 * cross-split log-sum-exp merge the reference sizes but never runs
 * (forward_gpu.cu:100, docs/reports/P7.md:13,32-34).
 *   q [batch][Hq][D] fp16, seq_lens device int32[batch] (keys 0..len-1),
 *   out [batch][Hq][D] fp16, kv_head = q_head / (Hq/Hkv),
 *   scale 1/sqrt(D) (decode_attention_split.cu:197).
 * num_splits: 0 = auto (see kvhp_decode_auto_splits), else the number of
 * equal KV chunks max_seq_len is cut into.
 * workspace: NULL = library-owned per-device buffer (allocated on first use,
 * so not capturable into a HIP graph); otherwise at least
 * kvhp_decode_workspace_bytes() bytes.  With more than one split the call is
 * two launches on `stream` (split kernel, then merge kernel).  Concurrent
 * calls sharing one workspace race. */
int kvhp_decode_attention(const void* q, const kvhp_kv_view* k_view,
                          const kvhp_kv_view* v_view, const int32_t* seq_lens,
                          void* out, int batch, int num_q_heads,
                          int num_kv_heads, int head_dim, int max_seq_len,
                          int num_splits, void* workspace,
                          size_t workspace_bytes, void* stream);

/* No counterpart in the reference: kvhp_decode_attention for callers that
 * cannot allocate device memory (code under HIP graph capture, serving
 * loops that forbid hipMalloc).  Same arguments and results as
 * kvhp_decode_attention with workspace = NULL, but the split partials live
 * in a static 16 MiB device array of the library (one per GPU, held until
 * the process ends) instead of an allocated buffer; the call allocates
 * nothing.  A plan whose partials exceed 16 MiB is rejected with
 * KVHP_ERR_WORKSPACE (config 3's auto plan needs 11.2 MB).  Every call on a
 * GPU shares that GPU's array: calls that overlap on one GPU (other streams
 * or threads) race.  Partials need no clearing: a call reads only the ones
 * it wrote.  The first call on a device resolves the array's address and
 * its kernels' occupancy (no allocation, no stream work): make that first
 * call, with the shapes to be captured, outside graph capture (a first call
 * under capture is refused with KVHP_ERR_INVALID, nothing enqueued); later
 * calls may be captured (tested: two calls in one graph, replays
 * bit-identical to eager kvhp_decode_attention). */
int kvhp_decode_attention_noalloc(const void* q, const kvhp_kv_view* k_view,
                                  const kvhp_kv_view* v_view, const int32_t* seq_lens,
                                  void* out, int batch, int num_q_heads, int num_kv_heads,
                                  int head_dim, int max_seq_len, int num_splits,
                                  void* stream);

/* The serving step's append_kv_cache + decode_gqa_split pair
 * (src/model/forward_gpu.cu:593-640: append the new K/V row at pos, then
 * attend over pos+1 keys) in one call on paged views:
 *   k_new / v_new [batch][Hkv][D] fp16 (one token per sequence), written to
 *   position positions[b] (device int32[batch]) of the pools through the
 *   views' block table, exactly as kvhp_paged_append_kv (same drop rules),
 *   then attention as kvhp_decode_attention over seq_lens[b] keys, the new
 *   row included when positions[b] < seq_lens[b].
 * Within the fast kernel's shapes the row is attended from registers and
 * written by the one workgroup that covers it (no separate append launch);
 * otherwise the append kernel runs first.  Workspace as for
 * kvhp_decode_attention. */
int kvhp_paged_append_decode(const void* q, const void* k_new, const void* v_new,
                             const kvhp_kv_view* k_view, const kvhp_kv_view* v_view,
                             const int32_t* positions, const int32_t* seq_lens, void* out,
                             int batch, int num_q_heads, int num_kv_heads, int head_dim,
                             int max_seq_len, int num_splits, void* workspace,
                             size_t workspace_bytes, void* stream);
/* The same pair on views of either kind: paged views as
 * kvhp_paged_append_decode; strided views (the reference KVCache layout,
 * src/runtime/kv_cache.cu:8-36 then decode_attention_split.cu:183-214) get
 * row positions[b] of sequence b written, positions outside
 * [0, max_seq_len) dropped as the reference append drops those past
 * max_seq.  One launch (plus the merge) within the fast kernel's shapes. */
int kvhp_append_decode(const void* q, const void* k_new, const void* v_new,
                       const kvhp_kv_view* k_view, const kvhp_kv_view* v_view,
                       const int32_t* positions, const int32_t* seq_lens, void* out, int batch,
                       int num_q_heads, int num_kv_heads, int head_dim, int max_seq_len,
                       int num_splits, void* workspace, size_t workspace_bytes, void* stream);

/* Replaces engine::cuda::decode_gqa (src/cuda/kernels.h:104-115,
 * src/cuda/decode_attention.cu:114-137): one sequence, head-major cache
 * [Hkv][max_seq][D], total_seq_len keys; routed to kvhp_decode_attention. */
int kvhp_decode_gqa(const void* q, const void* k_cache, const void* v_cache,
                    void* out, int total_seq_len, int num_q_heads,
                    int num_kv_heads, int max_seq, int head_dim, void* stream);

/* Replaces engine::cuda::flash_prefill_gqa (src/cuda/kernels.h:135-147,
 * src/cuda/flash_prefill.cu:214-240): causal attention over token-major
 * q [batch][S][Hq][D], k/v [batch][S][Hkv][D] -> out [batch][S][Hq][D]. */
int kvhp_flash_prefill(const void* q, const void* k, const void* v, void* out,
                       int64_t seq_len, int num_q_heads, int num_kv_heads,
                       int head_dim, int batch, void* stream);

/* flash_prefill_gqa that also writes each sequence's K/V rows into the paged
 * pool as it consumes them (the reference does this with a separate
 * append_kv_cache before attention, src/model/forward_gpu.cu:423-440).
 * Positions 0..S-1 of sequence b go through block_tables[b]. */
int kvhp_flash_prefill_paged(const void* q, const void* k, const void* v,
                             void* out, int64_t seq_len, int num_q_heads,
                             int num_kv_heads, int head_dim, int batch,
                             void* pool_k, void* pool_v,
                             const int32_t* block_tables, int max_pages,
                             int num_pages, void* stream);

/* Replaces engine::cuda::causal_gqa (src/cuda/kernels.h:71-87,
 * src/cuda/causal_attention.cu:131-143): batch-1 causal attention; routed to
 * the flash prefill kernel. */
int kvhp_causal_gqa(const void* q, const void* k, const void* v, void* out,
                    int64_t seq_len, int64_t num_q_heads, int64_t num_kv_heads,
                    int64_t head_dim, void* stream);

/* ---- Model operators around the KV-cache path (decoder-only model,
 * batch-1 decode).  fp16 tensors row-major; W [N][K] is the PyTorch linear
 * weight layout the reference uses (src/cuda/kernels.h:178-192). ---------- */

/* Replaces engine::cuda::gemv (src/cuda/kernels.h:207-217,
 * src/cuda/gemv.cu:29-63): y[n] = sum_k W[n][k] x[k], fp32 accumulation,
 * fp16 y. */
int kvhp_gemv(const void* W, const void* x, void* y, int N, int K, void* stream);
/* Replaces engine::cuda::gemv_residual (src/cuda/kernels.h:231-241):
 * y[n] = dot(W[n], x) + r[n]; r may alias y (in-place residual stream). */
int kvhp_gemv_residual(const void* W, const void* x, const void* r, void* y, int N, int K,
                       void* stream);
/* rmsnorm (src/cuda/kernels.h:24-32) fused into the following GEMV:
 * xn = fp16(x * rsqrt(mean(x^2) + eps) * norm_w), y = W xn, written to
 * exactly one of y16 (fp16) or y32 (fp32, the reference's fp32 logits,
 * kernels.h:194-205). */
int kvhp_rmsnorm_gemv(const void* W, const void* x, const void* norm_w, float eps, void* y16,
                      float* y32, int N, int K, void* stream);
/* rmsnorm + gate/up projections + swiglu (kernels.h:150-158) in one pass:
 * W_gate_up = [gate; up], [2N][K]; out[n] = silu(g) * u with g, u the fp16
 * projections of the normalised x. */
int kvhp_rmsnorm_gemv_swiglu(const void* W_gate_up, const void* x, const void* norm_w, float eps,
                             void* out, int N, int K, void* stream);
/* rmsnorm + fused q/k/v projection + apply_rope (kernels.h:57-70) +
 * append_kv_cache (src/runtime/kv_cache.h:80-91) for one decode token:
 * W_qkv = [Wq; Wk; Wv], [(Hq + 2 Hkv) D][K]; the token sits at position
 * seq_len[0] - 1 (device int32: "bump, then write at num_tokens - 1");
 * q_out [Hq][D] gets rotated q, rotated k and v go into page
 * block_table[pos/16] slot pos%16 of pools [Hkv][num_pages][16][D]. */
int kvhp_rmsnorm_qkv_rope_append(const void* W_qkv, const void* x, const void* norm_w, float eps,
                                 const int32_t* seq_len, float rope_theta, void* q_out,
                                 void* pool_k, void* pool_v, const int32_t* block_table,
                                 int max_pages, int num_pages, int num_q_heads, int num_kv_heads,
                                 int head_dim, int K, void* stream);
/* Batched decode projections: the four fused GEMVs above for `batch`
 * sequences at once (1 <= batch <= 32), x / outputs row-major [batch][...].
 * Each weight element is read once per call for all rows (a skinny GEMM on
 * v_mfma_f32_16x16x32_f16); epilogues and roundings as the batch-1 calls.
 * K must be 256*n (n <= 8), or 352*n (n <= 16) for kvhp_gemv_residual_rows;
 * head_dim a multiple of 32 for the QKV call; otherwise
 * KVHP_ERR_UNSUPPORTED.  The QKV call rotates row b at positions[b]
 * (device int32) and writes its k / v into page
 * block_tables[b][positions[b] / 16] (rows [batch][max_pages]); a negative
 * position marks an idle row (q written, nothing appended). */
int kvhp_gemv_residual_rows(const void* W, const void* x, const void* r, void* y, int N, int K,
                            int batch, void* stream);
/* No counterpart in the reference (its batched projections are library
 * GEMMs).  kvhp_gemv_residual_rows with a caller workspace: when the batch's
 * x exceeds 160 KB (batch*K > 81920, e.g. the down projection, K = 5632,
 * from 15 rows) and N % 16 == 0, the product is split over K into fp32
 * partials (kvhp_gemv_rows_workspace_bytes bytes) and summed by a second
 * launch, so that no CU loads all of x; the output is bit-identical to
 * kvhp_gemv_residual_rows.  Workspace bytes 0 (or workspace NULL): the
 * single-launch path.  r may alias y. */
size_t kvhp_gemv_rows_workspace_bytes(int N, int K, int batch);
int kvhp_gemv_residual_rows_ws(const void* W, const void* x, const void* r, void* y, int N,
                               int K, int batch, void* workspace, size_t workspace_bytes,
                               void* stream);
int kvhp_rmsnorm_gemv_rows(const void* W, const void* x, const void* norm_w, float eps, void* y16,
                           float* y32, int N, int K, int batch, void* stream);
int kvhp_rmsnorm_gemv_swiglu_rows(const void* W_gate_up, const void* x, const void* norm_w,
                                  float eps, void* out, int N, int K, int batch, void* stream);
int kvhp_rmsnorm_qkv_rope_append_rows(const void* W_qkv, const void* x, const void* norm_w,
                                      float eps, const int32_t* positions, float rope_theta,
                                      void* q_out, void* pool_k, void* pool_v,
                                      const int32_t* block_tables, int max_pages, int num_pages,
                                      int num_q_heads, int num_kv_heads, int head_dim, int K,
                                      int batch, void* stream);
/* No counterpart in the reference (its batched projections are library
 * GEMMs).  The batched projections above over weights pre-tiled for them:
 * kvhp_rows_tile_weights copies W (row-major, as the calls above take it)
 * into kvhp_rows_tiled_bytes bytes in which every 16-row tile keeps, per
 * 32-wide k step, the 64 MFMA lanes' 16-byte operands contiguous (rows in
 * the order the kernels pair them: SwiGLU gate/up rows, RoPE dimension
 * pairs), so one wave's weight load is 1 KB contiguous instead of 16 rows of
 * 64 bytes.  kind: KVHP_ROWS_PLAIN (the residual / fp16 / fp32 calls,
 * N rows), KVHP_ROWS_SWIGLU (W_gate_up, N gate rows then N up rows),
 * KVHP_ROWS_QKV (N ignored: (Hq + 2 Hkv) head_dim rows).  The *_tiled calls
 * take the tiled copy in place of W, with the arguments of their row-major
 * counterparts (kvhp_gemv_residual_rows_tiled that of _ws: workspace NULL or
 * 0 bytes for the single-launch path), and give bit-identical outputs.
 * Unsupported shapes (those the row-major calls refuse): size 0,
 * KVHP_ERR_UNSUPPORTED. */
#define KVHP_ROWS_PLAIN 0
#define KVHP_ROWS_SWIGLU 1
#define KVHP_ROWS_QKV 2
size_t kvhp_rows_tiled_bytes(int kind, int N, int K, int num_q_heads, int num_kv_heads,
                             int head_dim);
int kvhp_rows_tile_weights(int kind, const void* W, int N, int K, int num_q_heads,
                           int num_kv_heads, int head_dim, void* W_tiled, void* stream);
int kvhp_gemv_residual_rows_tiled(const void* W_tiled, const void* x, const void* r, void* y,
                                  int N, int K, int batch, void* workspace,
                                  size_t workspace_bytes, void* stream);
int kvhp_rmsnorm_gemv_rows_tiled(const void* W_tiled, const void* x, const void* norm_w,
                                 float eps, void* y16, float* y32, int N, int K, int batch,
                                 void* stream);
int kvhp_rmsnorm_gemv_swiglu_rows_tiled(const void* W_tiled, const void* x, const void* norm_w,
                                        float eps, void* out, int N, int K, int batch,
                                        void* stream);
int kvhp_rmsnorm_qkv_rope_append_rows_tiled(const void* W_tiled, const void* x,
                                            const void* norm_w, float eps,
                                            const int32_t* positions, float rope_theta,
                                            void* q_out, void* pool_k, void* pool_v,
                                            const int32_t* block_tables, int max_pages,
                                            int num_pages, int num_q_heads, int num_kv_heads,
                                            int head_dim, int K, int batch, void* stream);
/* Replaces engine::cuda::rmsnorm (kernels.h:24-32): rows x dim, fp32 math. */
int kvhp_rmsnorm(const void* x, const void* weight, void* out, int64_t rows, int64_t dim,
                 float eps, void* stream);
/* Replaces engine::cuda::apply_rope (kernels.h:57-70): half-split RoPE in
 * place on q [S][Hq][D], k [S][Hkv][D], positions start_pos.. */
int kvhp_apply_rope(void* q, void* k, int64_t seq_len, int64_t num_q_heads, int64_t num_kv_heads,
                    int64_t head_dim, int64_t start_pos, float rope_theta, void* stream);
/* Prefill helper: split a fused projection [S][(Hq + 2 Hkv) D] into
 * contiguous q [S][Hq][D], k, v [S][Hkv][D], with RoPE on q and k. */
int kvhp_split_qkv_rope(const void* qkv, int64_t seq_len, int num_q_heads, int num_kv_heads,
                        int head_dim, int64_t start_pos, float rope_theta, void* q, void* k,
                        void* v, void* stream);
/* Batched decode helper: as kvhp_split_qkv_rope for `rows` sequences, row r
 * rotated at positions[r] (device int32; negative = idle row, rotated as
 * position 0) -- the reference's per-token rope (rope.cu:8-57) at each
 * sequence's write position. */
int kvhp_split_qkv_rope_rows(const void* qkv, int64_t rows, int num_q_heads, int num_kv_heads,
                             int head_dim, const int32_t* positions, float rope_theta, void* q,
                             void* k, void* v, void* stream);
/* Replaces engine::cuda::swiglu (kernels.h:150-158): out = silu(g) * u. */
int kvhp_swiglu(const void* gate, const void* up, void* out, int64_t count, void* stream);
/* swiglu over rows of a fused [gate | up] buffer [rows][2n] -> out [rows][n]. */
int kvhp_swiglu_rows(const void* gate_up, void* out, int64_t rows, int64_t n, void* stream);
/* Replaces engine::cuda::embedding_lookup (kernels.h:12-20) with device
 * int32 ids (ids outside [0, vocab) give zero rows). */
int kvhp_embedding(const int32_t* token_ids, const void* table, void* out, int64_t n,
                   int64_t hidden, int64_t vocab, void* stream);
/* Greedy sampling on device (the reference's host argmax loop,
 * apps/generate.cpp:714-721): token = argmax of fp32 logits, lowest index
 * on ties, NaN never chosen.  Optional: log[*log_count] = token and
 * ++*log_count; ++*seq_len (the next step's "bump"). */
int kvhp_argmax(const float* logits, int64_t n, int32_t* token, int32_t* seq_len, int32_t* log,
                int32_t* log_count, void* stream);
/* Batched greedy sampling: tokens[r] = argmax of row r of logits [rows][n]
 * (same tie and NaN rules as kvhp_argmax); one workgroup per row. */
int kvhp_argmax_rows(const float* logits, int64_t rows, int64_t n, int32_t* tokens, void* stream);
/* Seeded N(0, std_dev) fp16 fill (synthetic weights): element i of stream
 * stream_id is a Box-Muller normal of two splitmix64 hashes of
 * (seed, stream_id, i). */
int kvhp_randn_f16(void* out, int64_t count, uint64_t seed, uint64_t stream_id, float std_dev,
                   void* stream);
/* Constant fp16 fill. */
int kvhp_fill_f16(void* out, int64_t count, float value, void* stream);

/* ---- Decoder-only model runner (config 5: Llama-style, batch 1), the
 * reference's model entry points prefill_gpu / decode_step_gpu
 * (src/model/forward_gpu.h:88-113) over this library's kernels.  Weights are
 * synthetic: every matrix N(0, 0.02) fp16 from kvhp_randn_f16 with the given
 * seed (one stream id per tensor, in creation order), RMSNorm weights 1; the
 * LM head is untied; no projection biases. ---------------------------------- */
typedef struct kvhp_llama_config {
    int vocab_size;
    int hidden_size;
    int num_layers;
    int num_q_heads;
    int num_kv_heads;
    int head_dim;
    int ffn_size;
    float rms_eps;
    float rope_theta;
    int reserved;
} kvhp_llama_config;

/* Tensor ids for kvhp_llama_tensor (layer < 0: model-level tensors). */
#define KVHP_LLAMA_EMBED 0       /* [V][H]                         */
#define KVHP_LLAMA_LM_HEAD 1     /* [V][H]                         */
#define KVHP_LLAMA_FINAL_NORM 2  /* [H]                            */
#define KVHP_LLAMA_ATTN_NORM 10  /* [H]                            */
#define KVHP_LLAMA_FFN_NORM 11   /* [H]                            */
#define KVHP_LLAMA_W_QKV 12      /* [(Hq + 2 Hkv) D][H]: q; k; v   */
#define KVHP_LLAMA_W_O 13        /* [H][Hq D]                      */
#define KVHP_LLAMA_W_GATE_UP 14  /* [2F][H]: gate; up              */
#define KVHP_LLAMA_W_DOWN 15     /* [H][F]                         */
#define KVHP_LLAMA_POOL_K 16     /* [Hkv][P][16][D] KV pages       */
#define KVHP_LLAMA_POOL_V 17

/* Allocate and initialise a model for contexts up to max_ctx tokens. */
int kvhp_llama_create(const kvhp_llama_config* config, uint64_t seed, int max_ctx,
                      void** model);
int kvhp_llama_destroy(void* model);
/* prefill_gpu (forward_gpu.h:93-101): n prompt ids (host), K/V of every
 * position into the pages; logits_out (host, V floats, may be NULL) of the
 * last position; *next_token = its greedy argmax. */
int kvhp_llama_prefill(void* model, const int32_t* tokens, int n, float* logits_out,
                       int32_t* next_token);
/* decode_step_gpu (forward_gpu.h:103-113): one token at the next position.
 * token < 0 continues from the last greedy token; token >= 0 replaces it
 * (teacher forcing).  logits_out (host) and *next_token as for prefill. */
int kvhp_llama_decode_step(void* model, int32_t token, float* logits_out, int32_t* next_token);
/* n_steps greedy decode steps entirely on the device (use_graph: captured
 * once as a HIP graph, replayed per step).  tokens_out (host) receives every
 * token generated since the prefill (its argmax first); *elapsed_ms the
 * device time of the n_steps steps. */
int kvhp_llama_generate(void* model, int n_steps, int use_graph, int32_t* tokens_out,
                        float* elapsed_ms);
/* Device pointer and element count of a model tensor (fp16). */
int kvhp_llama_tensor(void* model, int layer, int which, void** ptr, size_t* count);

/* ---- Batched serving over caller-owned pages: the reference runner
 * contract (docs/runner_interface.md:18-53; Runner.prefill / decode_step)
 * with the scheduler's page pool and block tables in the caller's hands.
 * pool: [num_layers][2][Hkv][num_pages][16][D] fp16 (engine::PagedKVCache's
 * raw_data() layout); block tables int32 rows of max_pages page ids (-1 =
 * none: reads clamp, writes are dropped).  The model's activation buffers
 * (max_ctx rows) are reused, so calls on one model must not overlap: issue
 * them on one stream, or synchronise between streams. */

/* prefill(seq) (runner_interface.md:20-33): the n prompt ids (host) run
 * through the model; the K/V of position t go to page block_table[t/16]
 * (device, one row) slot t%16 of every layer -- pass the write table
 * (engine::PagedKVCache::write_block_tables) so pages shared with other
 * sequences keep their cached K/V ("share" prefix mode).  The caller has
 * allocated pages for all n positions (n <= 16 * max_pages, n <= max_ctx).
 * logits_out (host, V floats, may be NULL) are those of the last position;
 * *next_token its greedy argmax.  Runs on `stream`; returns when done. */
int kvhp_llama_prefill_paged(void* model, const int32_t* tokens, int n, void* pool,
                             int num_pages, const int32_t* block_table, int max_pages,
                             float* logits_out, int32_t* next_token, void* stream);
/* prefill(seq) in the "full" prefix mode (runner_interface.md:30-33): the
 * first num_cached of the n prompt positions (0 < num_cached < n) already
 * have their K/V in the pages of block_table (a cached, possibly shared,
 * prefix); only positions [num_cached, n) run through the model, each
 * attending over the keys up to itself read through block_table, their K/V
 * appended through write_table (NULL: block_table; pass the write table,
 * shared pages -1, when a forwarded position lies in a shared page, e.g.
 * the last token of a fully cached prompt).  Outputs and preconditions as
 * kvhp_llama_prefill_paged. */
int kvhp_llama_prefill_cached(void* model, const int32_t* tokens, int n, int num_cached,
                              void* pool, int num_pages, const int32_t* block_table,
                              const int32_t* write_table, int max_pages, float* logits_out,
                              int32_t* next_token, void* stream);
/* decode_step(seqs) (runner_interface.md:37-53) for `batch` sequences
 * (batch <= max_ctx), all arguments device memory: row b embeds tokens[b],
 * appends its K/V at positions[b] through row b of block_tables [batch]
 * [max_pages] (-1: an idle row, nothing written), attends over seq_lens[b]
 * keys (<= max_seq_len; the caller has already bumped it, so positions[b] =
 * seq_lens[b] - 1), and ends in fp32 logits [batch][V] and greedy
 * next_tokens[batch] (lowest index on ties).  Up to 32 sequences run on the
 * fused batched projections (kvhp_*_rows_tiled: each weight read once per
 * step, from the model's tiled copy of it, which the first such step builds
 * on `stream` -- as large as the four projections and the LM head; weights
 * written through kvhp_llama_tensor after that are seen by batched steps once
 * kvhp_llama_reserve rebuilds the copies); larger batches on library GEMMs.
 * Asynchronous on `stream`. */
int kvhp_llama_decode_paged(void* model, const int32_t* tokens, int batch, void* pool,
                            int num_pages, const int32_t* block_tables, int max_pages,
                            const int32_t* positions, const int32_t* seq_lens, int max_seq_len,
                            float* logits, int32_t* next_tokens, void* stream);
/* Sizes the model's own decode buffers (split-attention partials, the
 * batched down projection's K-split partials) for every kvhp_llama_decode_paged
 * call with batch <= max_batch and max_seq_len <= max_seq_len, so that such
 * calls allocate nothing, and (max_batch > 1) builds or rebuilds the batched
 * projections' tiled weights from the current weights, synchronously.  No
 * reference counterpart (the reference sizes its
 * split buffer once at load, forward_gpu.cu:100).  A call that needs larger
 * buffers grows them (the old ones stay allocated until kvhp_llama_destroy,
 * so graphs captured earlier keep valid addresses); under HIP graph capture it
 * cannot, and returns KVHP_ERR_WORKSPACE having enqueued at most the step's
 * embedding lookup.  So: reserve before capturing decode_paged (batches up to
 * 32; larger batches run library GEMMs, which are not meant for capture).
 * kvhp_llama_prefill_paged / _cached synchronise and are never captured. */
int kvhp_llama_reserve(void* model, int max_batch, int max_seq_len);

#ifdef __cplusplus
}
#endif
#endif /* KVHP_C_H */
