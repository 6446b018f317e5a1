// kernels.h -- C++ attention entry points, reference names and signatures.
//
// Mirrors the attention part of engine::cuda (reference src/cuda/kernels.h
// :71-87, :99-147) over the C ABI in kvhp_c.h.  Arguments keep the
// reference's order and meaning; `cudaStream_t` becomes hipStream_t and
// `half` the 16-bit storage type of half.h.  A non-zero library status is
// thrown as std::runtime_error, as the reference's CUDA_CHECK does
// (src/common/cuda_utils.h:12-21).  All calls enqueue on `stream` and return
// without synchronising.
//
// The functions live in engine::hip; `engine::cuda` is an alias of it, so a
// caller written against the reference (`cuda::decode_gqa_split(...)`)
// compiles unchanged.
#pragma once

#include <cstdint>

#include "half.h"
#include "hip_utils.h"
#include "kv_view.h"
#include "kvhp_c.h"

namespace engine {
namespace hip {

// Largest split count the reference-signature decode_gqa_split uses with a
// caller split_buffer: the smallest buffer any reference caller allocates
// is kSplitBufferSplits * B * Hq * (D + 2) floats (test_attention.cpp:124;
// forward_gpu.cu:100 and bench_attention.cpp:52 allocate 16 splits' worth).
constexpr int kSplitBufferSplits = 8;

// Floats a caller split_buffer must hold for decode_gqa_split.
inline size_t decode_split_buffer_floats(int batch_size, int num_q_heads, int head_dim) {
    return (size_t)kSplitBufferSplits * batch_size * num_q_heads * (head_dim + 2);
}

// Causal GQA over token-major q [S][Hq][D], k/v [S][Hkv][D] -> out
// [S][Hq][D], scale 1/sqrt(D) (reference kernels.h:71-87).  Routed to the
// flash prefill kernel.
inline void causal_gqa(const half* q, const half* k, const half* v, half* out, int64_t seq_len,
                       int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                       Stream stream = nullptr) {
    KVHP_CHECK(kvhp_causal_gqa(q, k, v, out, seq_len, num_q_heads, num_kv_heads, head_dim,
                               stream));
}

// One-token decode over a head-major cache [Hkv][max_seq][D], attending to
// keys 0..total_seq_len-1 (reference kernels.h:99-115).
inline void decode_gqa(const half* q, const half* k_cache, const half* v_cache, half* out,
                       int total_seq_len, int num_q_heads, int num_kv_heads, int max_seq,
                       int head_dim, Stream stream = nullptr) {
    KVHP_CHECK(kvhp_decode_gqa(q, k_cache, v_cache, out, total_seq_len, num_q_heads,
                               num_kv_heads, max_seq, head_dim, stream));
}

// Batched split-K decode (reference kernels.h:117-133).  q [B][Hq][D],
// out [B][Hq][D], seq_lens device int32 [B]; k_view / v_view strided or
// paged.  split_buffer == nullptr: the library's per-device workspace and
// its automatic split count.  Otherwise split_buffer must hold
// decode_split_buffer_floats(B, Hq, D) floats and at most
// kSplitBufferSplits splits are used (the reference accepted the buffer but
// never used it, decode_attention_split.cu:183-214).  A sequence with
// seq_lens[b] <= 0 gets zeros (the reference leaves its rows unwritten).
// One-stream rule: with split_buffer == nullptr every call on a device
// shares that device's one library workspace, so calls on two streams that
// can overlap race on the split partials (the reference's single-stream use
// is safe); give each stream its own split_buffer (or decode_gqa_split_ex
// workspace) when decoding concurrently.  The workspace also grows by
// reallocating, so a call that needs more than any earlier one must not be
// under graph capture (decode_gqa_split_ex with a caller workspace never
// allocates).
inline void decode_gqa_split(const half* q, KVView k_view, KVView v_view, const int* seq_lens,
                             half* out, int batch_size, int num_q_heads, int num_kv_heads,
                             int head_dim, int max_seq_len, float* split_buffer = nullptr,
                             Stream stream = nullptr) {
    int splits = 0;
    size_t bytes = 0;
    if (split_buffer) {
        splits = kvhp_decode_auto_splits(batch_size, num_kv_heads, head_dim, max_seq_len);
        if (splits > kSplitBufferSplits) splits = kSplitBufferSplits;
        bytes = decode_split_buffer_floats(batch_size, num_q_heads, head_dim) * sizeof(float);
    }
    KVHP_CHECK(kvhp_decode_attention(q, k_view.c_view(), v_view.c_view(), seq_lens, out,
                                     batch_size, num_q_heads, num_kv_heads, head_dim,
                                     max_seq_len, splits, split_buffer, bytes, stream));
}

// decode_gqa_split with the split count and workspace explicit: num_splits
// 0 = automatic; workspace nullptr = library-owned, else at least
// decode_workspace_bytes(...) bytes.
inline size_t decode_workspace_bytes(int batch_size, int num_q_heads, int num_kv_heads,
                                     int head_dim, int max_seq_len, int num_splits = 0) {
    return kvhp_decode_workspace_bytes(batch_size, num_q_heads, num_kv_heads, head_dim,
                                       max_seq_len, num_splits);
}
inline void decode_gqa_split_ex(const half* q, const KVView& k_view, const KVView& v_view,
                                const int* seq_lens, half* out, int batch_size, int num_q_heads,
                                int num_kv_heads, int head_dim, int max_seq_len, int num_splits,
                                void* workspace, size_t workspace_bytes,
                                Stream stream = nullptr) {
    KVHP_CHECK(kvhp_decode_attention(q, k_view.c_view(), v_view.c_view(), seq_lens, out,
                                     batch_size, num_q_heads, num_kv_heads, head_dim,
                                     max_seq_len, num_splits, workspace, workspace_bytes,
                                     stream));
}

// Flash-style causal prefill over token-major activations q [B][S][Hq][D],
// k/v [B][S][Hkv][D] -> out [B][S][Hq][D] (reference kernels.h:135-147).
inline void flash_prefill_gqa(const half* q, const half* k, const half* v, half* out,
                              int64_t seq_len, int num_q_heads, int num_kv_heads, int head_dim,
                              int batch_size = 1, Stream stream = nullptr) {
    KVHP_CHECK(kvhp_flash_prefill(q, k, v, out, seq_len, num_q_heads, num_kv_heads, head_dim,
                                  batch_size, stream));
}

// flash_prefill_gqa that also stores every sequence's K/V rows 0..S-1 into
// the paged pools [Hkv][num_pages][16][D] through block_tables
// [B][max_pages] (the reference runs append_kv_cache before attention for
// this, forward_gpu.cu:423-440).
inline void flash_prefill_gqa_paged(const half* q, const half* k, const half* v, half* out,
                                    int64_t seq_len, int num_q_heads, int num_kv_heads,
                                    int head_dim, int batch_size, half* pool_k, half* pool_v,
                                    const int32_t* block_tables, int max_pages, int num_pages,
                                    Stream stream = nullptr) {
    KVHP_CHECK(kvhp_flash_prefill_paged(q, k, v, out, seq_len, num_q_heads, num_kv_heads,
                                        head_dim, batch_size, pool_k, pool_v, block_tables,
                                        max_pages, num_pages, stream));
}

// Paged append: token t of sequence b ([B][T][Hkv][D]) goes to position
// start_pos[b] + t (device int32 [B]) through block_tables [B][max_pages].
inline void paged_append_kv(const half* src_k, const half* src_v, half* pool_k, half* pool_v,
                            const int32_t* block_tables, int max_pages, const int32_t* start_pos,
                            int batch_size, int num_tokens, int num_kv_heads, int head_dim,
                            int num_pages, Stream stream = nullptr) {
    KVHP_CHECK(kvhp_paged_append_kv(src_k, src_v, pool_k, pool_v, block_tables, max_pages,
                                    start_pos, batch_size, num_tokens, num_kv_heads, head_dim,
                                    num_pages, stream));
}

// The serving step's append + decode in one call (kvhp_paged_append_decode):
// row b of k_new / v_new [B][Hkv][D] goes to position positions[b] through
// the views' block table, then decode attention over seq_lens[b] keys.
inline void paged_append_decode(const half* q, const half* k_new, const half* v_new,
                                const KVView& k_view, const KVView& v_view,
                                const int32_t* positions, const int32_t* seq_lens, half* out,
                                int batch_size, int num_q_heads, int num_kv_heads, int head_dim,
                                int max_seq_len, Stream stream = nullptr) {
    KVHP_CHECK(kvhp_paged_append_decode(q, k_new, v_new, k_view.c_view(), v_view.c_view(),
                                        positions, seq_lens, out, batch_size, num_q_heads,
                                        num_kv_heads, head_dim, max_seq_len, 0, nullptr, 0,
                                        stream));
}

// Paged gather into contiguous out [B][Hkv][max_len][D] (zeros past
// seq_lens[b]).
inline void paged_gather_kv(const half* pool_k, const half* pool_v, const int32_t* block_tables,
                            int max_pages, const int32_t* seq_lens, int batch_size,
                            int num_kv_heads, int head_dim, int num_pages, int max_len,
                            half* out_k, half* out_v, Stream stream = nullptr) {
    KVHP_CHECK(kvhp_paged_gather_kv(pool_k, pool_v, block_tables, max_pages, seq_lens,
                                    batch_size, num_kv_heads, head_dim, num_pages, max_len,
                                    out_k, out_v, stream));
}

}  // namespace hip

namespace cuda = hip;

}  // namespace engine
