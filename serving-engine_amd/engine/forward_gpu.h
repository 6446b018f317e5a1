// forward_gpu.h -- the reference's model entry points over engine::KVCache.
//
// prefill_gpu / decode_step_gpu keep the signatures of the reference's
// (src/model/forward_gpu.h:88-113): same parameter order and meaning, host
// fp32 logits of the last position returned (an empty vector when
// d_last_logits, a device buffer of vocab floats, receives them instead),
// the cache's current_seq_len set to the prompt length / current_pos + 1
// (forward_gpu.cu:494,683), and a std::runtime_error for a prompt longer
// than the activation buffers (:348-351).  The ordering contract is the
// reference's: position t's K/V are appended at t before position t
// attends over t + 1 keys.
//
// What backs them is this library's config-5 runner: the cache's
// [L][2][Hkv][max_seq][D] block is read as a page pool [L][2][Hkv][P][16][D]
// through an identity block table (byte-identical for max_seq = 16 P, so
// max_seq must be a multiple of 16), prefill runs kvhp_llama_prefill_paged
// (library GEMMs + the flash prefill kernel writing the pages) and a decode
// step kvhp_llama_decode_paged (fused GEMVs, split-K decode attention).
//
// Differences by design:
//   * ModelWeightsGPU holds synthetic weights (init_synthetic: every matrix
//     N(0, 0.02) in fp16 from the library's seeded generator, norms 1, no
//     projection biases) -- checkpoint loading (init_from_weights) is the
//     reference's loader, outside the KV-cache path; tie_word_embeddings
//     copies the embedding into the LM head.  It also owns the model's
//     activation rows (max_rows, the longest prompt one prefill takes).
//   * The BLAS handle is opaque and unused (the model owns its rocBLAS
//     handle); any pointer, or nullptr, may be passed where the reference
//     passes its cublasHandle_t.
//   * profile_records, when given, receives one record per call (the
//     call's device time), not one per kernel.
//   * Work runs on the default stream, as the reference's; calls on one
//     ModelWeightsGPU must not overlap.
#pragma once

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "config.h"
#include "hip_utils.h"
#include "kv_cache.h"
#include "kvhp_c.h"

namespace engine {

struct KernelRecord {
    std::string name;
    float ms;
};

class ModelWeightsGPU {
public:
    ModelWeightsGPU() = default;
    ~ModelWeightsGPU() { reset(); }
    ModelWeightsGPU(const ModelWeightsGPU&) = delete;
    ModelWeightsGPU& operator=(const ModelWeightsGPU&) = delete;
    ModelWeightsGPU(ModelWeightsGPU&& o) noexcept { *this = std::move(o); }
    ModelWeightsGPU& operator=(ModelWeightsGPU&& o) noexcept {
        if (this != &o) {
            reset();
            model_ = std::exchange(o.model_, nullptr);
            max_rows_ = std::exchange(o.max_rows_, 0);
            config_ = o.config_;
        }
        return *this;
    }

    // Synthetic weights of config's shape from `seed` (the same seed gives
    // the same weights as kvhp_llama_create).  max_rows <= 0 takes
    // config.max_position_embeddings.  Returns false on failure, as the
    // reference's init_from_weights (kvhp_last_error() has the reason).
    bool init_synthetic(const ModelConfig& config, uint64_t seed, int max_rows = 0) {
        reset();
        if (max_rows <= 0) max_rows = config.max_position_embeddings;
        const kvhp_llama_config c = config.to_c();
        if (kvhp_llama_create(&c, seed, max_rows, &model_) != KVHP_OK) {
            model_ = nullptr;
            return false;
        }
        if (config.tie_word_embeddings) {
            void *embed = nullptr, *head = nullptr;
            size_t n_embed = 0, n_head = 0;
            if (kvhp_llama_tensor(model_, -1, KVHP_LLAMA_EMBED, &embed, &n_embed) != KVHP_OK ||
                kvhp_llama_tensor(model_, -1, KVHP_LLAMA_LM_HEAD, &head, &n_head) != KVHP_OK ||
                hipMemcpy(head, embed, n_embed * sizeof(half), hipMemcpyDeviceToDevice) !=
                    hipSuccess) {
                reset();
                return false;
            }
        }
        config_ = c;
        max_rows_ = max_rows;
        return true;
    }

    void* handle() const { return model_; }
    int max_rows() const { return max_rows_; }
    const kvhp_llama_config& c_config() const { return config_; }

private:
    void reset() {
        if (model_) kvhp_llama_destroy(model_);
        model_ = nullptr;
        max_rows_ = 0;
    }
    void* model_ = nullptr;
    int max_rows_ = 0;
    kvhp_llama_config config_{};
};

// Per-call device staging of the two entry points (the reference's
// ActivationBuffersGPU, forward_gpu.h:44-64, keeps its activations here;
// this build's live with the model).  logits holds one row of vocab floats.
struct ActivationBuffersGPU {
    DeviceBuffer<float> logits;       // [vocab_size] fp32
    DeviceBuffer<int32_t> step;       // token, position, seq_len, next token
    DeviceBuffer<int32_t> block_table;// identity page table of the cache
    int64_t max_seq = 0;

    void allocate(const ModelConfig& config, int64_t max_seq_len) {
        if (max_seq_len <= 0)
            throw std::invalid_argument("ActivationBuffersGPU::allocate: max_seq_len must be positive");
        logits.allocate((size_t)config.vocab_size);
        step.allocate(4);
        block_table.reset();
        max_seq = max_seq_len;
    }
};

namespace detail {

inline void check_model(const ModelConfig& config, const ModelWeightsGPU& weights,
                        const ActivationBuffersGPU& buffers, const KVCache& kv, const char* what) {
    const kvhp_llama_config c = config.to_c();
    const kvhp_llama_config& w = weights.c_config();
    if (!weights.handle())
        throw std::logic_error(std::string(what) + ": weights not initialised");
    if (c.vocab_size != w.vocab_size || c.hidden_size != w.hidden_size ||
        c.num_layers != w.num_layers || c.num_q_heads != w.num_q_heads ||
        c.num_kv_heads != w.num_kv_heads || c.head_dim != w.head_dim ||
        c.ffn_size != w.ffn_size)
        throw std::invalid_argument(std::string(what) + ": config differs from the weights' shape");
    if (buffers.max_seq <= 0 || buffers.logits.size() < (size_t)c.vocab_size)
        throw std::logic_error(std::string(what) + ": activation buffers not allocated");
    if (kv.num_layers() != c.num_layers || kv.num_kv_heads() != c.num_kv_heads ||
        kv.head_dim() != c.head_dim)
        throw std::invalid_argument(std::string(what) + ": KV cache shape differs from the model");
    if (kv.max_seq() <= 0 || kv.max_seq() % KVHP_PAGE_SIZE != 0)
        throw std::invalid_argument(std::string(what) + ": KV cache max_seq " +
                                    std::to_string(kv.max_seq()) + " is not a multiple of " +
                                    std::to_string(KVHP_PAGE_SIZE));
}

// Identity block table over the cache's max_seq / 16 pages.
inline const int32_t* identity_table(ActivationBuffersGPU& buffers, int pages) {
    if (buffers.block_table.size() != (size_t)pages) {
        std::vector<int32_t> ident(pages);
        for (int i = 0; i < pages; ++i) ident[i] = i;
        buffers.block_table.allocate(pages);
        buffers.block_table.copy_from_host(ident.data(), ident.size());
    }
    return buffers.block_table.data();
}

inline std::vector<float> finish(const ModelConfig& config, ActivationBuffersGPU& buffers,
                                 float* d_last_logits) {
    std::vector<float> out;
    if (!d_last_logits) {
        out.resize(config.vocab_size);
        buffers.logits.copy_to_host(out.data(), out.size());
    }
    return out;
}

}  // namespace detail

// Prompt forward: K/V of positions [0, S) into the cache, logits of the
// last position (forward_gpu.h:88-101).
inline std::vector<float> prefill_gpu(const std::vector<int64_t>& token_ids,
                                      const ModelConfig& config, const ModelWeightsGPU& weights,
                                      ActivationBuffersGPU& buffers, KVCache& kv_cache,
                                      const void* blas_handle, float* d_last_logits = nullptr,
                                      std::vector<KernelRecord>* profile_records = nullptr) {
    (void)blas_handle;
    detail::check_model(config, weights, buffers, kv_cache, "prefill_gpu");
    const int64_t S = static_cast<int64_t>(token_ids.size());
    if (S > buffers.max_seq)
        throw std::runtime_error("prefill_gpu: seq_len " + std::to_string(S) +
                                 " exceeds max_seq " + std::to_string(buffers.max_seq));
    if (S <= 0) throw std::invalid_argument("prefill_gpu: empty prompt");
    if (S > weights.max_rows() || S > kv_cache.max_seq())
        throw std::runtime_error("prefill_gpu: seq_len " + std::to_string(S) +
                                 " exceeds the model's rows or the cache");
    std::vector<int32_t> ids(S);
    for (int64_t i = 0; i < S; ++i) {
        if (token_ids[i] < 0 || token_ids[i] >= config.vocab_size)
            throw std::out_of_range("prefill_gpu: token id " + std::to_string(token_ids[i]));
        ids[i] = static_cast<int32_t>(token_ids[i]);
    }
    const int pages = kv_cache.max_seq() / KVHP_PAGE_SIZE;
    const int32_t* bt = detail::identity_table(buffers, pages);
    std::unique_ptr<HipTimer> timer;
    if (profile_records) {
        timer.reset(new HipTimer);
        timer->start();
    }
    std::vector<float> host(config.vocab_size);
    int32_t next = 0;
    KVHP_CHECK(kvhp_llama_prefill_paged(weights.handle(), ids.data(), (int)S, kv_cache.raw_data(),
                                        pages, bt, pages, host.data(), &next, nullptr));
    if (profile_records) {
        timer->stop();
        profile_records->push_back({"prefill", timer->elapsed_ms()});
    }
    kv_cache.set_current_seq_len(static_cast<int>(S));
    float* target = d_last_logits ? d_last_logits : buffers.logits.data();
    HIP_CHECK(hipMemcpy(target, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice));
    if (d_last_logits) return {};
    return host;
}

// One token at current_pos: its K/V appended there, attention over
// current_pos + 1 keys, logits of the position (forward_gpu.h:103-113).
inline std::vector<float> decode_step_gpu(int64_t token_id, int current_pos,
                                          const ModelConfig& config,
                                          const ModelWeightsGPU& weights,
                                          ActivationBuffersGPU& buffers, KVCache& kv_cache,
                                          const void* blas_handle, float* d_last_logits = nullptr,
                                          std::vector<KernelRecord>* profile_records = nullptr) {
    (void)blas_handle;
    detail::check_model(config, weights, buffers, kv_cache, "decode_step_gpu");
    if (token_id < 0 || token_id >= config.vocab_size)
        throw std::out_of_range("decode_step_gpu: token id " + std::to_string(token_id));
    if (current_pos < 0 || current_pos >= kv_cache.max_seq())
        throw std::out_of_range("decode_step_gpu: position " + std::to_string(current_pos) +
                                " outside the cache's " + std::to_string(kv_cache.max_seq()));
    const int pages = kv_cache.max_seq() / KVHP_PAGE_SIZE;
    const int32_t* bt = detail::identity_table(buffers, pages);
    const int32_t step[3] = {static_cast<int32_t>(token_id), current_pos, current_pos + 1};
    buffers.step.copy_from_host(step, 3);
    const int32_t* d = buffers.step.data();
    float* target = d_last_logits ? d_last_logits : buffers.logits.data();
    std::unique_ptr<HipTimer> timer;
    if (profile_records) {
        timer.reset(new HipTimer);
        timer->start();
    }
    KVHP_CHECK(kvhp_llama_decode_paged(weights.handle(), d, 1, kv_cache.raw_data(), pages, bt,
                                       pages, d + 1, d + 2, kv_cache.max_seq(), target,
                                       buffers.step.data() + 3, nullptr));
    if (profile_records) {
        timer->stop();
        profile_records->push_back({"decode_step", timer->elapsed_ms()});
    }
    kv_cache.set_current_seq_len(current_pos + 1);
    return detail::finish(config, buffers, d_last_logits);
}

}  // namespace engine
