// ref_forward_shim.cpp -- C entry point over the reference's own CPU model
// forward (src/model/forward_cpu.h:42-52).
//
// TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile together with the
// reference sources src/model/forward_cpu.cpp, src/cpu/ops.cpp and
// src/loader/safetensors.cpp where they lie (never copied) into
// oracle/_ref/libref_forward.so, which tests use to pin the composition of
// oracle/llama_oracle.py (layer order, residuals, RoPE positions, GQA map).
//
// Weights arrive as one fp32 buffer, per layer in the order
//   input_layernorm[H], post_attention_layernorm[H], q[H*H], k[kvd*H],
//   v[kvd*H], o[H*H], gate[F*H], up[F*H], down[H*F]
// after embed[V*H] and final_norm[H]; projection biases are zero (the
// reference adds them, the Llama-style model has none) and the LM head is
// the embedding (the reference ties them).
#include "src/model/forward_cpu.h"

#include <cstring>

extern "C" int ref_forward_cpu(const int64_t* ids, int64_t S, int V, int H, int F, int L,
                               int Hq, int Hkv, int D, float eps, float theta,
                               const float* w, float* logits) {
    if (Hq * D != H) return -1;  // the reference's q buffer is [S][H]
    engine::ModelConfig c;
    c.vocab_size = V;
    c.hidden_size = H;
    c.intermediate_size = F;
    c.num_hidden_layers = L;
    c.num_attention_heads = Hq;
    c.num_key_value_heads = Hkv;
    c.head_dim = D;
    c.rms_norm_eps = eps;
    c.rope_theta = theta;
    const int64_t kvd = (int64_t)Hkv * D;
    engine::ModelWeightsFP32 m;
    auto take = [&](std::vector<float>& dst, int64_t n) {
        dst.assign(w, w + n);
        w += n;
    };
    take(m.embed_tokens, (int64_t)V * H);
    take(m.final_norm, H);
    m.layers.resize(L);
    for (auto& l : m.layers) {
        take(l.input_layernorm, H);
        take(l.post_attention_layernorm, H);
        take(l.q_proj_weight, (int64_t)H * H);
        take(l.k_proj_weight, kvd * H);
        take(l.v_proj_weight, kvd * H);
        take(l.o_proj_weight, (int64_t)H * H);
        take(l.gate_proj_weight, (int64_t)F * H);
        take(l.up_proj_weight, (int64_t)F * H);
        take(l.down_proj_weight, (int64_t)H * F);
        l.q_proj_bias.assign(H, 0.f);
        l.k_proj_bias.assign(kvd, 0.f);
        l.v_proj_bias.assign(kvd, 0.f);
    }
    std::vector<int64_t> tok(ids, ids + S);
    const std::vector<float> out = engine::forward_cpu(tok, c, m, "");
    std::memcpy(logits, out.data(), out.size() * sizeof(float));
    return 0;
}
