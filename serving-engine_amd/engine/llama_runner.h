// llama_runner.h -- the reference runner contract over PagedKVCache.
//
// Runner.prefill / Runner.decode_step (reference docs/runner_interface.md
// :18-53; the model entry points prefill_gpu / decode_step_gpu of
// src/model/forward_gpu.h:88-113) for a decoder-only model with synthetic
// weights (kvhp_llama_create), served over a PagedKVCache whose layer count,
// KV heads and head dim match the model:
//
//   * prefill(cache, slot, prompt, ..., num_cached): the scheduler has
//     already set the slot's length to the prompt length (pages reserved;
//     the runner allocates nothing and leaves the length alone).  K/V go
//     through the cache's write table, so pages the slot shares with another
//     sequence keep their cached K/V.  num_cached = 0 recomputes the whole
//     prompt ("share" prefix mode, :30-33); num_cached > 0 (the tokens
//     share_prefix() returned) forwards only the rest, which attends to the
//     cached prefix from the pages ("full" mode); num_cached may not exceed
//     the tokens the slot took over (PagedKVCache::cached_tokens), since
//     those positions are read, never written.  Returns the greedy first
//     token.
//   * decode_step(cache, batch, tokens): "bump, then write at num_tokens - 1"
//     for every active slot in [0, batch) (PagedKVCache::begin_decode_step,
//     which throws if a write would land on a shared page, :51), then one
//     batched step (up to 32 slots on the batched projections: each weight
//     read once for all of them), attention per slot over its own block
//     table.  Returns the greedy next token per slot (-1 for inactive
//     slots).
//
// Calls on one runner must not overlap (they share activation buffers).
#pragma once

#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "hip_utils.h"
#include "kv_cache.h"
#include "kvhp_c.h"

namespace engine {

class LlamaRunner {
public:
    // max_rows bounds the prompt length of one prefill and the batch of one
    // decode step (the activation buffers' rows).
    LlamaRunner(const kvhp_llama_config& config, uint64_t seed, int max_rows) : config_(config) {
        KVHP_CHECK(kvhp_llama_create(&config, seed, max_rows, &model_));
        max_rows_ = max_rows;
    }
    ~LlamaRunner() {
        if (model_) kvhp_llama_destroy(model_);
    }
    LlamaRunner(const LlamaRunner&) = delete;
    LlamaRunner& operator=(const LlamaRunner&) = delete;

    int prefill(PagedKVCache& cache, int slot, const std::vector<int32_t>& prompt,
                std::vector<float>* logits = nullptr, Stream stream = nullptr,
                int num_cached = 0) {
        check_cache(cache);
        if (slot < 0 || slot >= cache.max_batch())
            throw std::out_of_range("LlamaRunner::prefill: slot " + std::to_string(slot));
        if (prompt.empty() || cache.seq_len(slot) != (int)prompt.size())
            throw std::logic_error("LlamaRunner::prefill: the slot's length must already be the "
                                   "prompt length (" + std::to_string(prompt.size()) + ")");
        if (num_cached < 0 || num_cached > (int)prompt.size())
            throw std::invalid_argument("LlamaRunner::prefill: num_cached " +
                                        std::to_string(num_cached));
        // positions below num_cached are read, not written: they must hold
        // K/V taken over by share_prefix
        if (num_cached > cache.cached_tokens(slot))
            throw std::invalid_argument("LlamaRunner::prefill: num_cached " +
                                        std::to_string(num_cached) + " exceeds the slot's " +
                                        std::to_string(cache.cached_tokens(slot)) +
                                        " shared-prefix tokens");
        cache.sync(stream);
        if (logits) logits->resize(config_.vocab_size);
        int32_t tok = -1;
        const size_t row = (size_t)slot * cache.max_pages_per_seq();
        if (num_cached > 0) {
            // a fully cached prompt still forwards its last token
            const int first = std::min(num_cached, (int)prompt.size() - 1);
            KVHP_CHECK(kvhp_llama_prefill_cached(
                model_, prompt.data(), (int)prompt.size(), first, cache.raw_data(),
                cache.num_pages(), cache.block_tables() + row, cache.write_block_tables() + row,
                cache.max_pages_per_seq(), logits ? logits->data() : nullptr, &tok, stream));
        } else {
            KVHP_CHECK(kvhp_llama_prefill_paged(
                model_, prompt.data(), (int)prompt.size(), cache.raw_data(), cache.num_pages(),
                cache.write_block_tables() + row, cache.max_pages_per_seq(),
                logits ? logits->data() : nullptr, &tok, stream));
        }
        return tok;
    }

    // tokens[b]: the last token of slot b (ignored for inactive slots).
    // logits (optional): [batch][vocab] fp32 on return.
    std::vector<int32_t> decode_step(PagedKVCache& cache, int batch,
                                     const std::vector<int32_t>& tokens,
                                     std::vector<float>* logits = nullptr,
                                     Stream stream = nullptr) {
        check_cache(cache);
        if (batch <= 0 || batch > max_rows_ || (int)tokens.size() < batch)
            throw std::invalid_argument("LlamaRunner::decode_step: batch " + std::to_string(batch));
        cache.begin_decode_step(batch);
        int max_len = 1;
        for (int s = 0; s < batch; ++s) max_len = std::max(max_len, cache.seq_len(s));
        cache.sync(stream);
        if (tokens_.size() < (size_t)batch) {
            tokens_.allocate(batch);
            next_.allocate(batch);
        }
        if (logits_.size() < (size_t)batch * config_.vocab_size)
            logits_.allocate((size_t)batch * config_.vocab_size);
        HIP_CHECK(hipMemcpyAsync(tokens_.data(), tokens.data(), (size_t)batch * 4,
                                 hipMemcpyHostToDevice, stream));
        KVHP_CHECK(kvhp_llama_decode_paged(model_, tokens_.data(), batch, cache.raw_data(),
                                           cache.num_pages(), cache.block_tables(),
                                           cache.max_pages_per_seq(), cache.write_positions(),
                                           cache.seq_lens(), max_len, logits_.data(),
                                           next_.data(), stream));
        std::vector<int32_t> next(batch);
        HIP_CHECK(hipMemcpyAsync(next.data(), next_.data(), (size_t)batch * 4,
                                 hipMemcpyDeviceToHost, stream));
        if (logits) {
            logits->resize((size_t)batch * config_.vocab_size);
            HIP_CHECK(hipMemcpyAsync(logits->data(), logits_.data(), logits->size() * 4,
                                     hipMemcpyDeviceToHost, stream));
        }
        HIP_CHECK(hipStreamSynchronize(stream));
        for (int s = 0; s < batch; ++s)
            if (cache.seq_len(s) == 0) next[s] = -1;
        return next;
    }

    void* handle() const { return model_; }
    const kvhp_llama_config& config() const { return config_; }

private:
    void check_cache(const PagedKVCache& cache) const {
        if (cache.num_layers() != config_.num_layers || cache.num_kv_heads() != config_.num_kv_heads ||
            cache.head_dim() != config_.head_dim)
            throw std::invalid_argument("LlamaRunner: the cache's layers / KV heads / head dim "
                                        "differ from the model's");
    }

    kvhp_llama_config config_;
    void* model_ = nullptr;
    int max_rows_ = 0;
    DeviceBuffer<int32_t> tokens_, next_;
    DeviceBuffer<float> logits_;
};

}  // namespace engine
