// config.h -- model configuration of the C++ API.
//
// ModelConfig mirrors engine::ModelConfig (reference src/model/config.h:9-25)
// field for field, with the reference's defaults, so code that fills one
// for the reference compiles unchanged.  llama_1b() gives the BASELINE
// config-5 model (Llama-style 1.1B).  to_c() maps it onto the C ABI's
// kvhp_llama_config.  Loading a config from a file (ModelConfig::from_file)
// is the reference's loader, not part of the KV-cache path, and is not
// provided.
#pragma once

#include <string>

#include "kvhp_c.h"

namespace engine {

struct ModelConfig {
    std::string model_type = "qwen2";
    int vocab_size = 151936;
    int hidden_size = 896;
    int intermediate_size = 4864;
    int num_hidden_layers = 24;
    int num_attention_heads = 14;
    int num_key_value_heads = 2;
    int head_dim = 64;
    int max_position_embeddings = 32768;
    float rms_norm_eps = 1e-6f;
    float rope_theta = 1000000.0f;
    bool tie_word_embeddings = true;
    std::string torch_dtype = "bfloat16";

    // 22 layers, hidden 2048, 32 q / 4 KV heads of 64, SwiGLU 5632, vocab
    // 32000, RMSNorm eps 1e-5, RoPE theta 1e4, untied LM head, fp16.
    static ModelConfig llama_1b() {
        ModelConfig c;
        c.model_type = "llama";
        c.vocab_size = 32000;
        c.hidden_size = 2048;
        c.intermediate_size = 5632;
        c.num_hidden_layers = 22;
        c.num_attention_heads = 32;
        c.num_key_value_heads = 4;
        c.head_dim = 64;
        c.max_position_embeddings = 2048;
        c.rms_norm_eps = 1e-5f;
        c.rope_theta = 10000.0f;
        c.tie_word_embeddings = false;
        c.torch_dtype = "float16";
        return c;
    }

    kvhp_llama_config to_c() const {
        kvhp_llama_config c{};
        c.vocab_size = vocab_size;
        c.hidden_size = hidden_size;
        c.num_layers = num_hidden_layers;
        c.num_q_heads = num_attention_heads;
        c.num_kv_heads = num_key_value_heads;
        c.head_dim = head_dim;
        c.ffn_size = intermediate_size;
        c.rms_eps = rms_norm_eps;
        c.rope_theta = rope_theta;
        return c;
    }
};

}  // namespace engine
