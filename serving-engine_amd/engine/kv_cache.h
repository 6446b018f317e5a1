// kv_cache.h -- KV cache owners of the C++ API.
//
// KVCache mirrors engine::KVCache (reference src/runtime/kv_cache.h:12-73)
// member for member: one zeroed fp16 allocation laid out
// [num_layers][2 (K, V)][num_kv_heads][max_seq][head_dim], the same pointer
// arithmetic, host-side current_seq_len.  append_kv_cache mirrors
// engine::cuda::append_kv_cache (kv_cache.h:76-91).
//
// PagedKVCache is the paged form the reference plans (src/cuda/kv_view.h
// :9-10) and its runner contract describes (docs/runner_interface.md
// :37-53, 81-84): per (layer, K|V) a pool [num_kv_heads][num_pages][16]
// [head_dim] of fp16 pages, int32 block tables [max_batch][max_pages] and
// int32 seq_lens [max_batch], with a host free list of pages.  Under the
// identity block table one sequence's pool is byte-identical to KVCache's
// [num_kv_heads][max_seq][head_dim] block for max_seq = 16 * num_pages.
// Pages carry reference counts: share_prefix() lets a sequence reuse another's
// full prefix pages (the runner contract's prefix sharing,
// docs/runner_interface.md:30-33); a decode write into a shared page throws,
// as the reference runner asserts (:51), and prefill writes go through a
// write table in which shared pages are -1, so they are never overwritten
// ("share" mode, :33).
#pragma once

#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "half.h"
#include "hip_utils.h"
#include "kernels.h"
#include "kv_view.h"
#include "kvhp_c.h"

namespace engine {

class KVCache {
public:
    KVCache() = default;
    KVCache(int num_layers, int num_kv_heads, int head_dim, int max_seq) {
        allocate(num_layers, num_kv_heads, head_dim, max_seq);
    }

    void allocate(int num_layers, int num_kv_heads, int head_dim, int max_seq) {
        num_layers_ = num_layers;
        num_kv_heads_ = num_kv_heads;
        head_dim_ = head_dim;
        max_seq_ = max_seq;
        data_.allocate((size_t)num_layers * 2 * num_kv_heads * max_seq * head_dim);
        data_.zero();
        current_seq_len_ = 0;
    }

    half* get_layer_ptr(int layer_idx, int is_v) { return data_.data() + layer_offset(layer_idx, is_v); }
    const half* get_layer_ptr(int layer_idx, int is_v) const {
        return data_.data() + layer_offset(layer_idx, is_v);
    }
    half* get_head_ptr(int layer_idx, int is_v, int kv_head) {
        return data_.data() + head_offset(layer_idx, is_v, kv_head);
    }
    const half* get_head_ptr(int layer_idx, int is_v, int kv_head) const {
        return data_.data() + head_offset(layer_idx, is_v, kv_head);
    }

    int num_layers() const { return num_layers_; }
    int num_kv_heads() const { return num_kv_heads_; }
    int head_dim() const { return head_dim_; }
    int max_seq() const { return max_seq_; }
    int current_seq_len() const { return current_seq_len_; }
    void set_current_seq_len(int len) { current_seq_len_ = len; }

    half* raw_data() { return data_.data(); }
    const half* raw_data() const { return data_.data(); }

private:
    size_t layer_offset(int l, int is_v) const {
        return ((size_t)l * 2 + is_v) * num_kv_heads_ * max_seq_ * head_dim_;
    }
    size_t head_offset(int l, int is_v, int h) const {
        return (((size_t)l * 2 + is_v) * num_kv_heads_ + h) * max_seq_ * head_dim_;
    }

    int num_layers_ = 0;
    int num_kv_heads_ = 0;
    int head_dim_ = 0;
    int max_seq_ = 0;
    int current_seq_len_ = 0;
    DeviceBuffer<half> data_;
};

namespace hip {

// Copies src [num_tokens][Hkv][D] into dst head bases [Hkv][max_seq][D] at
// positions start_pos.. (positions >= max_seq dropped).
inline void append_kv_cache(const half* src_k, const half* src_v, half* dst_k_head_base,
                            half* dst_v_head_base, int num_tokens, int start_pos,
                            int num_kv_heads, int max_seq, int head_dim,
                            Stream stream = nullptr) {
    KVHP_CHECK(kvhp_append_kv(src_k, src_v, dst_k_head_base, dst_v_head_base, num_tokens,
                              start_pos, num_kv_heads, max_seq, head_dim, stream));
}

}  // namespace hip

class PagedKVCache {
public:
    static constexpr int kPage = KVHP_PAGE_SIZE;

    PagedKVCache() = default;
    PagedKVCache(int num_layers, int num_kv_heads, int head_dim, int num_pages, int max_batch,
                 int max_pages_per_seq) {
        allocate(num_layers, num_kv_heads, head_dim, num_pages, max_batch, max_pages_per_seq);
    }
    ~PagedKVCache() { release_staging(); }
    PagedKVCache(const PagedKVCache&) = delete;
    PagedKVCache& operator=(const PagedKVCache&) = delete;

    // Pages that fit in `bytes` of pool for this model shape (K and V of
    // every layer).
    static int pages_for_bytes(size_t bytes, int num_layers, int num_kv_heads, int head_dim) {
        const size_t per_page = (size_t)num_layers * 2 * num_kv_heads * kPage * head_dim * sizeof(half);
        const size_t n = bytes / per_page;
        return n > (size_t)INT32_MAX ? INT32_MAX : (int)n;
    }

    void allocate(int num_layers, int num_kv_heads, int head_dim, int num_pages, int max_batch,
                  int max_pages_per_seq) {
        if (num_layers <= 0 || num_kv_heads <= 0 || head_dim <= 0 || num_pages <= 0 ||
            max_batch <= 0 || max_pages_per_seq <= 0)
            throw std::invalid_argument("PagedKVCache::allocate: sizes must be positive");
        release_staging();
        num_layers_ = num_layers;
        num_kv_heads_ = num_kv_heads;
        head_dim_ = head_dim;
        num_pages_ = num_pages;
        max_batch_ = max_batch;
        max_pages_ = max_pages_per_seq;
        pool_.allocate((size_t)num_layers * 2 * num_kv_heads * num_pages * kPage * head_dim);
        pool_.zero();
        // one device block: tables [max_batch][max_pages], seq_lens [max_batch],
        // write positions [max_batch], write tables [max_batch][max_pages]
        meta_words_ = 2 * (size_t)max_batch * max_pages_per_seq + 2 * (size_t)max_batch;
        meta_.allocate(meta_words_);
        void* p = nullptr;
        HIP_CHECK(hipHostMalloc(&p, meta_words_ * sizeof(int32_t), hipHostMallocDefault));
        staging_ = static_cast<int32_t*>(p);
        HIP_CHECK(hipEventCreateWithFlags(&staged_, hipEventDisableTiming));
        tables_.assign((size_t)max_batch * max_pages_per_seq, -1);
        lens_.assign(max_batch, 0);
        pos_.assign(max_batch, -1);
        pages_used_.assign(max_batch, 0);
        cached_.assign(max_batch, 0);
        active_.assign(max_batch, false);
        free_pages_.resize(num_pages);
        for (int i = 0; i < num_pages; ++i) free_pages_[i] = num_pages - 1 - i;  // pop 0 first
        refs_.assign(num_pages, 0);
        std::copy(tables_.begin(), tables_.end(), staging_);
        std::fill(staging_ + tables_.size(), staging_ + meta_words_, 0);
        std::fill(staging_ + tables_.size() + 2 * (size_t)max_batch, staging_ + meta_words_, -1);
        HIP_CHECK(hipMemcpy(meta_.data(), staging_, meta_words_ * sizeof(int32_t),
                            hipMemcpyHostToDevice));
    }

    // --- device side ------------------------------------------------------
    // Pool of one layer's K (is_v = 0) or V: [Hkv][num_pages][16][D].
    half* get_layer_ptr(int layer, int is_v) { return pool_.data() + layer_offset(layer, is_v); }
    const half* get_layer_ptr(int layer, int is_v) const {
        return pool_.data() + layer_offset(layer, is_v);
    }
    const int32_t* block_tables() const { return meta_.data(); }
    const int32_t* seq_lens() const { return meta_.data() + (size_t)max_batch_ * max_pages_; }
    const int32_t* write_positions() const { return seq_lens() + max_batch_; }
    // Block tables for writes: as block_tables(), with pages that more than
    // one sequence holds set to -1 (writes there are dropped).
    const int32_t* write_block_tables() const { return write_positions() + max_batch_; }
    hip::KVView k_view(int layer) const { return view(layer, 0); }
    hip::KVView v_view(int layer) const { return view(layer, 1); }

    // --- host page management (the scheduler's side of the contract) -------
    int add_sequence() {
        for (int s = 0; s < max_batch_; ++s) {
            if (!active_[s]) {
                active_[s] = true;
                lens_[s] = 0;
                pos_[s] = -1;
                return s;
            }
        }
        throw std::runtime_error("PagedKVCache::add_sequence: all batch slots in use");
    }
    // Ensures pages back positions [0, num_tokens) of `slot`.
    void reserve(int slot, int num_tokens) {
        check_slot(slot);
        const int need = (num_tokens + kPage - 1) / kPage;
        if (need > max_pages_)
            throw std::runtime_error("PagedKVCache::reserve: " + std::to_string(num_tokens) +
                                     " tokens exceed max_pages_per_seq");
        if (need - pages_used_[slot] > (int)free_pages_.size())
            throw std::runtime_error("PagedKVCache::reserve: out of pages");
        while (pages_used_[slot] < need) {
            const int32_t page = free_pages_.back();
            free_pages_.pop_back();
            refs_[page] = 1;
            tables_[(size_t)slot * max_pages_ + pages_used_[slot]] = page;
            ++pages_used_[slot];
        }
    }
    // Returns the slot's pages to the free list.
    void release(int slot) {
        check_slot(slot);
        for (int i = 0; i < pages_used_[slot]; ++i) {
            int32_t& e = tables_[(size_t)slot * max_pages_ + i];
            if (--refs_[e] == 0) free_pages_.push_back(e);
            e = -1;
        }
        pages_used_[slot] = 0;
        cached_[slot] = 0;
        lens_[slot] = 0;
        pos_[slot] = -1;
        active_[slot] = false;
    }
    void set_seq_len(int slot, int len) {
        check_slot(slot);
        if (len < 0)
            throw std::invalid_argument("PagedKVCache::set_seq_len: negative length");
        reserve(slot, len);
        lens_[slot] = len;
    }
    // Prefix sharing: `dst` (an active slot holding no pages) takes the
    // full pages covering the first num_tokens positions of `src` (a partial
    // last page is never shared, so later writes stay private) and starts
    // with that many cached tokens.  Returns the shared token count.
    int share_prefix(int dst, int src, int num_tokens) {
        check_slot(dst);
        check_slot(src);
        if (dst == src || !active_[dst] || !active_[src])
            throw std::invalid_argument("PagedKVCache::share_prefix: two distinct active slots needed");
        if (pages_used_[dst] != 0)
            throw std::logic_error("PagedKVCache::share_prefix: destination already holds pages");
        if (num_tokens < 0 || num_tokens > lens_[src])
            throw std::out_of_range("PagedKVCache::share_prefix: prefix longer than the source");
        const int n = num_tokens / kPage;
        for (int i = 0; i < n; ++i) {
            const int32_t page = tables_[(size_t)src * max_pages_ + i];
            tables_[(size_t)dst * max_pages_ + i] = page;
            ++refs_[page];
        }
        pages_used_[dst] = n;
        lens_[dst] = n * kPage;
        cached_[dst] = n * kPage;
        return n * kPage;
    }
    // Leading positions of `slot` whose K/V came from share_prefix (0 after
    // release): the most a cached-prefix prefill may take as already cached.
    int cached_tokens(int slot) const { return cached_.at(slot); }
    // Sequences holding physical page `page` (0: free).
    int page_refs(int page) const { return refs_.at(page); }
    int seq_len(int slot) const { return lens_.at(slot); }
    int pages_used(int slot) const { return pages_used_.at(slot); }
    int free_page_count() const { return (int)free_pages_.size(); }
    const int32_t* host_block_table(int slot) const { return tables_.data() + (size_t)slot * max_pages_; }

    // One decode step for slots [0, batch): "bump, then write at
    // num_tokens - 1" (docs/runner_interface.md:37-53): every active slot's
    // length grows by one, a page is added when it crosses a page boundary,
    // and its write position becomes the new length - 1.  Inactive slots get
    // length 0 and write position -1 (their appends are dropped).  A write
    // into a page that another sequence also holds throws, as the reference
    // runner asserts (docs/runner_interface.md:51); so does a step the free
    // pages cannot cover.  Either check runs before any slot changes.
    void begin_decode_step(int batch) {
        check_batch(batch);
        int new_pages = 0;
        for (int s = 0; s < batch; ++s) {
            if (!active_[s]) continue;
            const int idx = lens_[s] / kPage;   // page of the write position
            if (idx >= max_pages_)
                throw std::runtime_error("PagedKVCache::begin_decode_step: slot " + std::to_string(s) +
                                         " exceeds max_pages_per_seq");
            if (idx >= pages_used_[s])
                new_pages += idx + 1 - pages_used_[s];
            else if (refs_[tables_[(size_t)s * max_pages_ + idx]] > 1)
                throw std::logic_error("PagedKVCache::begin_decode_step: slot " + std::to_string(s) +
                                       " would write into a shared page");
        }
        if (new_pages > (int)free_pages_.size())
            throw std::runtime_error("PagedKVCache::begin_decode_step: out of pages");
        for (int s = 0; s < batch; ++s) {
            if (!active_[s]) {
                pos_[s] = -1;
                continue;
            }
            reserve(s, lens_[s] + 1);
            pos_[s] = lens_[s];
            lens_[s] += 1;
        }
    }
    // Write positions for a prefill of `num_tokens` tokens starting at each
    // slot's current length; lengths grow by num_tokens.  Writes go through
    // write_block_tables(), so positions on shared pages are left as cached.
    void begin_prefill(int batch, int num_tokens) {
        check_batch(batch);
        if (num_tokens < 0)
            throw std::invalid_argument("PagedKVCache::begin_prefill: negative token count");
        for (int s = 0; s < batch; ++s) {
            if (!active_[s]) {
                pos_[s] = -1;
                continue;
            }
            reserve(s, lens_[s] + num_tokens);
            pos_[s] = lens_[s];
            lens_[s] += num_tokens;
        }
    }

    // Enqueues the host tables, lengths and write positions to the device on
    // `stream`.  The host copies may be changed as soon as this returns (the
    // pinned staging buffer is reused only after the previous upload ended).
    void sync(Stream stream = nullptr) {
        HIP_CHECK(hipEventSynchronize(staged_));
        std::copy(tables_.begin(), tables_.end(), staging_);
        std::copy(lens_.begin(), lens_.end(), staging_ + tables_.size());
        std::copy(pos_.begin(), pos_.end(), staging_ + tables_.size() + max_batch_);
        int32_t* wt = staging_ + tables_.size() + 2 * (size_t)max_batch_;
        for (size_t i = 0; i < tables_.size(); ++i)
            wt[i] = tables_[i] >= 0 && refs_[tables_[i]] > 1 ? -1 : tables_[i];
        HIP_CHECK(hipMemcpyAsync(meta_.data(), staging_, meta_words_ * sizeof(int32_t),
                                 hipMemcpyHostToDevice, stream));
        HIP_CHECK(hipEventRecord(staged_, stream));
    }

    // --- per-layer hot path ---------------------------------------------------
    // Appends src [batch][num_tokens][Hkv][D] at each slot's write position.
    void append(int layer, const half* src_k, const half* src_v, int batch, int num_tokens,
                Stream stream = nullptr) {
        check_layer(layer);
        check_batch(batch);
        hip::paged_append_kv(src_k, src_v, get_layer_ptr(layer, 0), get_layer_ptr(layer, 1),
                             write_block_tables(), max_pages_, write_positions(), batch,
                             num_tokens, num_kv_heads_, head_dim_, num_pages_, stream);
    }
    // Decode attention of q [batch][Hq][D] over each slot's seq_len keys.
    void decode(int layer, const half* q, half* out, int batch, int num_q_heads, int max_seq_len,
                Stream stream = nullptr) const {
        check_layer(layer);
        check_batch(batch);
        hip::decode_gqa_split(q, k_view(layer), v_view(layer), seq_lens(), out, batch,
                              num_q_heads, num_kv_heads_, head_dim_, max_seq_len, nullptr, stream);
    }

    // One decode token per slot: append k_new / v_new [batch][Hkv][D] at each
    // slot's write position, then attend q over each slot's seq_len keys,
    // in one call (append and decode of the same step, fused).
    void append_decode(int layer, const half* k_new, const half* v_new, const half* q, half* out,
                       int batch, int num_q_heads, int max_seq_len, Stream stream = nullptr) {
        check_layer(layer);
        check_batch(batch);
        hip::paged_append_decode(q, k_new, v_new, k_view(layer), v_view(layer),
                                 write_positions(), seq_lens(), out, batch, num_q_heads,
                                 num_kv_heads_, head_dim_, max_seq_len, stream);
    }

    int num_layers() const { return num_layers_; }
    int num_kv_heads() const { return num_kv_heads_; }
    int head_dim() const { return head_dim_; }
    int num_pages() const { return num_pages_; }
    int max_batch() const { return max_batch_; }
    int max_pages_per_seq() const { return max_pages_; }
    half* raw_data() { return pool_.data(); }
    size_t pool_bytes() const { return pool_.size_bytes(); }

private:
    size_t layer_offset(int l, int is_v) const {
        return ((size_t)l * 2 + is_v) * num_kv_heads_ * (size_t)num_pages_ * kPage * head_dim_;
    }
    hip::KVView view(int layer, int is_v) const {
        return hip::paged_view(get_layer_ptr(layer, is_v), num_pages_, head_dim_, block_tables(),
                               max_pages_);
    }
    void check_slot(int slot) const {
        if (slot < 0 || slot >= max_batch_)
            throw std::out_of_range("PagedKVCache: slot " + std::to_string(slot));
    }
    // Device tables, lengths and write positions hold max_batch rows.
    void check_batch(int batch) const {
        if (batch < 0 || batch > max_batch_)
            throw std::out_of_range("PagedKVCache: batch " + std::to_string(batch) +
                                    " outside 0.." + std::to_string(max_batch_));
    }
    void check_layer(int layer) const {
        if (layer < 0 || layer >= num_layers_)
            throw std::out_of_range("PagedKVCache: layer " + std::to_string(layer));
    }
    void release_staging() {
        if (staged_) {
            (void)hipEventSynchronize(staged_);
            (void)hipEventDestroy(staged_);
            staged_ = nullptr;
        }
        if (staging_) {
            (void)hipHostFree(staging_);
            staging_ = nullptr;
        }
    }

    int num_layers_ = 0, num_kv_heads_ = 0, head_dim_ = 0, num_pages_ = 0;
    int max_batch_ = 0, max_pages_ = 0;
    DeviceBuffer<half> pool_;
    DeviceBuffer<int32_t> meta_;
    size_t meta_words_ = 0;
    int32_t* staging_ = nullptr;
    hipEvent_t staged_ = nullptr;
    std::vector<int32_t> tables_, lens_, pos_;
    std::vector<int> pages_used_;
    std::vector<int> cached_;
    std::vector<bool> active_;
    std::vector<int32_t> free_pages_;
    std::vector<int> refs_;
};

}  // namespace engine
