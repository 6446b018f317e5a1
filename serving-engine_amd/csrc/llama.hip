// llama.hip -- decoder-only model runner over the KV-cache path (config 5:
// Llama-style 1.1B, batch-1 greedy generation).
//
// Follows the reference's model entry points prefill_gpu / decode_step_gpu
// (src/model/forward_gpu.h:88-113, forward_gpu.cu:329-707) with the layer
// order of its CPU forward (src/model/forward_cpu.cpp:99-173): embedding;
// per layer RMSNorm -> q/k/v projections -> RoPE -> KV append -> causal GQA
// attention -> o projection + residual -> RMSNorm -> gate/up -> SwiGLU ->
// down projection + residual; final RMSNorm -> LM head (fp32 logits).
// Differences by design: no projection biases (Llama), an untied LM head,
// q/k/v and gate/up weights stored fused, a paged KV cache (per layer pools
// [Hkv][P][16][D], pages handed out in order), the decode step entirely on
// the device (token, position and KV append never leave the GPU, greedy
// argmax on device) so that it can be captured once in a HIP graph and
// replayed per token.
//
// Prefill projections are library GEMMs (rocBLAS, fp16 in, fp32 compute,
// fp16 out; the o and down projections accumulate into the residual stream
// with beta = 1); attention is the flash prefill kernel, which also writes
// the prompt's K/V pages.  Decode uses the fused GEMV kernels of
// model_ops.hip and the split-K decode attention of decode.hip.
//
// Synthetic weights: every matrix N(0, 0.02) in fp16 from the seeded
// device generator (kvhp_randn_f16, one stream id per tensor); RMSNorm
// weights are 1.
#include "kvhp_internal.h"

#include <rocblas/rocblas.h>

#include <cstring>
#include <memory>
#include <vector>

namespace kvhp {
namespace {

constexpr float kInitStd = 0.02f;

struct Layer {
    f16* attn_norm = nullptr;  // [H]
    f16* ffn_norm = nullptr;   // [H]
    f16* w_qkv = nullptr;      // [(Hq + 2Hkv) D][H]
    f16* w_o = nullptr;        // [H][Hq D]
    f16* w_gate_up = nullptr;  // [2F][H]
    f16* w_down = nullptr;     // [H][F]
    f16* pool_k = nullptr;     // [Hkv][P][16][D]
    f16* pool_v = nullptr;
};

struct Model {
    kvhp_llama_config c{};
    int max_ctx = 0;
    int P = 0;                 // pages per layer pool
    hipStream_t stream = nullptr;
    rocblas_handle blas = nullptr;
    std::vector<void*> allocs;
    f16* embed = nullptr;      // [V][H]
    f16* final_norm = nullptr; // [H]
    f16* lm_head = nullptr;    // [V][H]
    std::vector<Layer> layers;
    int32_t* bt = nullptr;     // [P] identity page order
    // prefill activations, sized for max_ctx rows
    f16 *hidden = nullptr, *norm = nullptr, *qkv = nullptr, *q = nullptr, *k = nullptr,
        *v = nullptr, *attn = nullptr, *gu = nullptr, *act = nullptr;
    // decode activations
    f16 *x = nullptr, *q1 = nullptr, *attn1 = nullptr, *act1 = nullptr;
    float* logits = nullptr;   // [V]
    int32_t* tokens = nullptr; // [max_ctx] prompt ids
    int32_t* state = nullptr;  // [0] seq_len, [1] current token, [2] log count
    int32_t* log = nullptr;    // [max_ctx] generated tokens
    void* ws = nullptr;        // decode attention workspace
    size_t ws_bytes = 0;
    int prompt_len = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;

    ~Model() {
        if (graph_exec) (void)hipGraphExecDestroy(graph_exec);
        if (graph) (void)hipGraphDestroy(graph);
        if (blas) rocblas_destroy_handle(blas);
        if (stream) (void)hipStreamSynchronize(stream);
        for (void* p : allocs) (void)hipFree(p);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

int alloc(Model& m, size_t bytes, void** out) {
    void* p = nullptr;
    KVHP_HIP(hipMalloc(&p, bytes < 256 ? 256 : bytes), "hipMalloc(model)");
    m.allocs.push_back(p);
    *out = p;
    return KVHP_OK;
}

template <typename T>
int alloc_n(Model& m, size_t n, T** out) {
    void* p = nullptr;
    const int rc = alloc(m, n * sizeof(T), &p);
    *out = static_cast<T*>(p);
    return rc;
}

#define KVHP_TRY(expr)            \
    do {                          \
        const int rc_ = (expr);   \
        if (rc_) return rc_;      \
    } while (0)

int blas_check(rocblas_status st, const char* what) {
    if (st != rocblas_status_success)
        return fail(KVHP_ERR_HIP, "%s: rocBLAS status %d", what, static_cast<int>(st));
    return KVHP_OK;
}

// C[M][N] (+)= A[M][K] W[N][K]^T, row-major, fp16 in/out, fp32 compute.
int linear(Model& m, const f16* A, const f16* W, f16* C, int M, int N, int K, bool accumulate) {
    const float alpha = 1.f, beta = accumulate ? 1.f : 0.f;
    return blas_check(rocblas_gemm_ex(m.blas, rocblas_operation_transpose,
                                      rocblas_operation_none, N, M, K, &alpha, W,
                                      rocblas_datatype_f16_r, K, A, rocblas_datatype_f16_r, K,
                                      &beta, C, rocblas_datatype_f16_r, N, C,
                                      rocblas_datatype_f16_r, N, rocblas_datatype_f32_r,
                                      rocblas_gemm_algo_standard, 0, 0),
                      "linear");
}

kvhp_kv_view pool_view(const Model& m, const f16* pool) {
    kvhp_kv_view v{};
    v.data = pool;
    v.stride_b = 0;
    v.stride_h = (int64_t)m.P * kPage * m.c.head_dim;
    v.stride_s = m.c.head_dim;
    v.stride_d = 1;
    v.block_table = m.bt;
    v.max_pages = m.P;
    v.page_size = kPage;
    v.num_pages = m.P;
    return v;
}

// One decode step on the device: token m.state[1] at position m.state[0] - 1.
// The greedy argmax that ends the prefill and every step also writes the
// chosen token's embedding row into m.x, so a step that continues from it
// starts without an embedding launch; embed_token re-reads m.state[1]
// (after the caller replaced the token).
int decode_step_kernels(Model& m, bool embed_token) {
    const kvhp_llama_config& c = m.c;
    const int H = c.hidden_size, D = c.head_dim, Hq = c.num_q_heads, Hkv = c.num_kv_heads;
    void* s = m.stream;
    if (embed_token) KVHP_TRY(kvhp_embedding(m.state + 1, m.embed, m.x, 1, H, c.vocab_size, s));
    for (const Layer& L : m.layers) {
        KVHP_TRY(kvhp_rmsnorm_qkv_rope_append(L.w_qkv, m.x, L.attn_norm, c.rms_eps, m.state,
                                              c.rope_theta, m.q1, L.pool_k, L.pool_v, m.bt, m.P,
                                              m.P, Hq, Hkv, D, H, s));
        const kvhp_kv_view kv = pool_view(m, L.pool_k), vv = pool_view(m, L.pool_v);
        KVHP_TRY(kvhp_decode_attention(m.q1, &kv, &vv, m.state, m.attn1, 1, Hq, Hkv, D, m.max_ctx,
                                       0, m.ws, m.ws_bytes, s));
        KVHP_TRY(kvhp_gemv_residual(L.w_o, m.attn1, m.x, m.x, H, Hq * D, s));
        KVHP_TRY(kvhp_rmsnorm_gemv_swiglu(L.w_gate_up, m.x, L.ffn_norm, c.rms_eps, m.act1,
                                          c.ffn_size, H, s));
        KVHP_TRY(kvhp_gemv_residual(L.w_down, m.act1, m.x, m.x, H, c.ffn_size, s));
    }
    KVHP_TRY(kvhp_rmsnorm_gemv(m.lm_head, m.x, m.final_norm, c.rms_eps, nullptr, m.logits,
                               c.vocab_size, H, s));
    return argmax_embed(m.logits, c.vocab_size, m.state + 1, m.state, m.log, m.state + 2, m.embed,
                        H, m.x, static_cast<hipStream_t>(s));
}

}  // namespace
}  // namespace kvhp

using namespace kvhp;

extern "C" int kvhp_llama_create(const kvhp_llama_config* cfg, uint64_t seed, int max_ctx,
                                 void** model) {
    clear_error();
    KVHP_REQUIRE(cfg && model, KVHP_ERR_INVALID, "llama_create: null argument");
    const kvhp_llama_config& c = *cfg;
    KVHP_REQUIRE(c.vocab_size > 0 && c.hidden_size > 0 && c.num_layers > 0 && c.num_q_heads > 0 &&
                     c.num_kv_heads > 0 && c.num_q_heads % c.num_kv_heads == 0 &&
                     c.head_dim > 0 && c.head_dim % 16 == 0 && c.ffn_size > 0 && max_ctx > 0,
                 KVHP_ERR_INVALID, "llama_create: bad configuration");
    KVHP_REQUIRE(c.num_q_heads * c.head_dim == c.hidden_size, KVHP_ERR_UNSUPPORTED,
                 "llama_create: num_q_heads * head_dim must equal hidden_size");
    auto m = std::make_unique<Model>();
    m->c = c;
    m->max_ctx = max_ctx;
    m->P = (max_ctx + kPage - 1) / kPage;
    KVHP_HIP(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking), "hipStreamCreate");
    KVHP_TRY(blas_check(rocblas_create_handle(&m->blas), "rocblas_create_handle"));
    KVHP_TRY(blas_check(rocblas_set_stream(m->blas, m->stream), "rocblas_set_stream"));

    const int H = c.hidden_size, D = c.head_dim, Hq = c.num_q_heads, Hkv = c.num_kv_heads;
    const int F = c.ffn_size, V = c.vocab_size, S = max_ctx;
    const int NQKV = (Hq + 2 * Hkv) * D;
    void* s = m->stream;
    uint64_t tensor_id = 0;
    auto randn = [&](f16** p, size_t n) {
        KVHP_TRY(alloc_n(*m, n, p));
        return kvhp_randn_f16(*p, (int64_t)n, seed, ++tensor_id, kInitStd, s);
    };
    auto ones = [&](f16** p, size_t n) {
        KVHP_TRY(alloc_n(*m, n, p));
        return kvhp_fill_f16(*p, (int64_t)n, 1.f, s);
    };
    KVHP_TRY(randn(&m->embed, (size_t)V * H));
    KVHP_TRY(randn(&m->lm_head, (size_t)V * H));
    KVHP_TRY(ones(&m->final_norm, H));
    m->layers.resize(c.num_layers);
    const size_t pool = (size_t)Hkv * m->P * kPage * D;
    for (Layer& L : m->layers) {
        KVHP_TRY(ones(&L.attn_norm, H));
        KVHP_TRY(ones(&L.ffn_norm, H));
        KVHP_TRY(randn(&L.w_qkv, (size_t)NQKV * H));
        KVHP_TRY(randn(&L.w_o, (size_t)H * Hq * D));
        KVHP_TRY(randn(&L.w_gate_up, (size_t)2 * F * H));
        KVHP_TRY(randn(&L.w_down, (size_t)H * F));
        KVHP_TRY(alloc_n(*m, pool, &L.pool_k));
        KVHP_TRY(alloc_n(*m, pool, &L.pool_v));
        KVHP_HIP(hipMemsetAsync(L.pool_k, 0, pool * 2, m->stream), "hipMemsetAsync(pool)");
        KVHP_HIP(hipMemsetAsync(L.pool_v, 0, pool * 2, m->stream), "hipMemsetAsync(pool)");
    }
    // identity block table: page i holds positions 16i .. 16i+15
    KVHP_TRY(alloc_n(*m, m->P, &m->bt));
    {
        std::vector<int32_t> ident(m->P);
        for (int i = 0; i < m->P; ++i) ident[i] = i;
        KVHP_HIP(hipMemcpyAsync(m->bt, ident.data(), ident.size() * 4, hipMemcpyHostToDevice,
                                m->stream),
                 "hipMemcpyAsync(block table)");
        KVHP_HIP(hipStreamSynchronize(m->stream), "hipStreamSynchronize");
    }
    KVHP_TRY(alloc_n(*m, (size_t)S * H, &m->hidden));
    KVHP_TRY(alloc_n(*m, (size_t)S * H, &m->norm));
    KVHP_TRY(alloc_n(*m, (size_t)S * NQKV, &m->qkv));
    KVHP_TRY(alloc_n(*m, (size_t)S * Hq * D, &m->q));
    KVHP_TRY(alloc_n(*m, (size_t)S * Hkv * D, &m->k));
    KVHP_TRY(alloc_n(*m, (size_t)S * Hkv * D, &m->v));
    KVHP_TRY(alloc_n(*m, (size_t)S * Hq * D, &m->attn));
    KVHP_TRY(alloc_n(*m, (size_t)S * 2 * F, &m->gu));
    KVHP_TRY(alloc_n(*m, (size_t)S * F, &m->act));
    KVHP_TRY(alloc_n(*m, H, &m->x));
    KVHP_TRY(alloc_n(*m, (size_t)Hq * D, &m->q1));
    KVHP_TRY(alloc_n(*m, (size_t)Hq * D, &m->attn1));
    KVHP_TRY(alloc_n(*m, F, &m->act1));
    KVHP_TRY(alloc_n(*m, V, &m->logits));
    KVHP_TRY(alloc_n(*m, S, &m->tokens));
    KVHP_TRY(alloc_n(*m, 4, &m->state));
    KVHP_TRY(alloc_n(*m, S, &m->log));
    m->ws_bytes = kvhp_decode_workspace_bytes(1, Hq, Hkv, D, max_ctx, 0);
    KVHP_TRY(alloc(*m, m->ws_bytes, &m->ws));
    KVHP_HIP(hipStreamSynchronize(m->stream), "hipStreamSynchronize(create)");
    *model = m.release();
    return KVHP_OK;
}

extern "C" int kvhp_llama_destroy(void* model) {
    clear_error();
    delete static_cast<Model*>(model);
    return KVHP_OK;
}

extern "C" int kvhp_llama_prefill(void* model, const int32_t* tokens, int n, float* logits_out,
                                  int32_t* next_token) {
    clear_error();
    KVHP_REQUIRE(model && tokens && n > 0, KVHP_ERR_INVALID, "llama_prefill: bad arguments");
    Model& m = *static_cast<Model*>(model);
    const kvhp_llama_config& c = m.c;
    KVHP_REQUIRE(n < m.max_ctx, KVHP_ERR_INVALID, "llama_prefill: %d tokens leave no room in %d",
                 n, m.max_ctx);
    const int H = c.hidden_size, D = c.head_dim, Hq = c.num_q_heads, Hkv = c.num_kv_heads;
    const int F = c.ffn_size, NQKV = (Hq + 2 * Hkv) * D;
    void* s = m.stream;
    KVHP_HIP(hipMemcpyAsync(m.tokens, tokens, (size_t)n * 4, hipMemcpyHostToDevice, m.stream),
             "hipMemcpyAsync(tokens)");
    // state: seq_len = n (bumped to n+1 by the argmax), log count 0
    const int32_t st[4] = {n, 0, 0, 0};
    KVHP_HIP(hipMemcpyAsync(m.state, st, sizeof st, hipMemcpyHostToDevice, m.stream),
             "hipMemcpyAsync(state)");
    KVHP_TRY(kvhp_embedding(m.tokens, m.embed, m.hidden, n, H, c.vocab_size, s));
    for (const Layer& L : m.layers) {
        KVHP_TRY(kvhp_rmsnorm(m.hidden, L.attn_norm, m.norm, n, H, c.rms_eps, s));
        KVHP_TRY(linear(m, m.norm, L.w_qkv, m.qkv, n, NQKV, H, false));
        KVHP_TRY(kvhp_split_qkv_rope(m.qkv, n, Hq, Hkv, D, 0, c.rope_theta, m.q, m.k, m.v, s));
        KVHP_TRY(kvhp_flash_prefill_paged(m.q, m.k, m.v, m.attn, n, Hq, Hkv, D, 1, L.pool_k,
                                          L.pool_v, m.bt, m.P, m.P, s));
        KVHP_TRY(linear(m, m.attn, L.w_o, m.hidden, n, H, Hq * D, true));
        KVHP_TRY(kvhp_rmsnorm(m.hidden, L.ffn_norm, m.norm, n, H, c.rms_eps, s));
        KVHP_TRY(linear(m, m.norm, L.w_gate_up, m.gu, n, 2 * F, H, false));
        KVHP_TRY(kvhp_swiglu_rows(m.gu, m.act, n, F, s));
        KVHP_TRY(linear(m, m.act, L.w_down, m.hidden, n, H, F, true));
    }
    // last position only: the decode residual stream continues from it
    KVHP_HIP(hipMemcpyAsync(m.x, m.hidden + (size_t)(n - 1) * H, (size_t)H * 2,
                            hipMemcpyDeviceToDevice, m.stream),
             "hipMemcpyAsync(last row)");
    KVHP_TRY(kvhp_rmsnorm_gemv(m.lm_head, m.x, m.final_norm, c.rms_eps, nullptr, m.logits,
                               c.vocab_size, H, s));
    KVHP_TRY(argmax_embed(m.logits, c.vocab_size, m.state + 1, m.state, m.log, m.state + 2,
                          m.embed, H, m.x, static_cast<hipStream_t>(s)));
    if (logits_out)
        KVHP_HIP(hipMemcpyAsync(logits_out, m.logits, (size_t)c.vocab_size * 4,
                                hipMemcpyDeviceToHost, m.stream),
                 "hipMemcpyAsync(logits)");
    int32_t host_state[4];
    KVHP_HIP(hipMemcpyAsync(host_state, m.state, sizeof host_state, hipMemcpyDeviceToHost,
                            m.stream),
             "hipMemcpyAsync(state)");
    KVHP_HIP(hipStreamSynchronize(m.stream), "hipStreamSynchronize(prefill)");
    if (next_token) *next_token = host_state[1];
    m.prompt_len = n;
    return KVHP_OK;
}

extern "C" int kvhp_llama_decode_step(void* model, int32_t token, float* logits_out,
                                      int32_t* next_token) {
    clear_error();
    KVHP_REQUIRE(model, KVHP_ERR_INVALID, "llama_decode_step: null model");
    Model& m = *static_cast<Model*>(model);
    int32_t st[4];
    KVHP_HIP(hipMemcpyAsync(st, m.state, sizeof st, hipMemcpyDeviceToHost, m.stream),
             "hipMemcpyAsync(state)");
    KVHP_HIP(hipStreamSynchronize(m.stream), "hipStreamSynchronize");
    KVHP_REQUIRE(m.prompt_len > 0, KVHP_ERR_INVALID, "llama_decode_step: no prefill yet");
    KVHP_REQUIRE(st[0] <= m.max_ctx, KVHP_ERR_INVALID, "llama_decode_step: context of %d full",
                 m.max_ctx);
    if (token >= 0)  // teacher forcing: replace the greedy token of the last step
        KVHP_HIP(hipMemcpyAsync(m.state + 1, &token, 4, hipMemcpyHostToDevice, m.stream),
                 "hipMemcpyAsync(token)");
    KVHP_TRY(decode_step_kernels(m, token >= 0));
    if (logits_out)
        KVHP_HIP(hipMemcpyAsync(logits_out, m.logits, (size_t)m.c.vocab_size * 4,
                                hipMemcpyDeviceToHost, m.stream),
                 "hipMemcpyAsync(logits)");
    KVHP_HIP(hipMemcpyAsync(st, m.state, sizeof st, hipMemcpyDeviceToHost, m.stream),
             "hipMemcpyAsync(state)");
    KVHP_HIP(hipStreamSynchronize(m.stream), "hipStreamSynchronize(decode)");
    if (next_token) *next_token = st[1];
    return KVHP_OK;
}

extern "C" int kvhp_llama_generate(void* model, int n_steps, int use_graph, int32_t* tokens_out,
                                   float* elapsed_ms) {
    clear_error();
    KVHP_REQUIRE(model && n_steps >= 0, KVHP_ERR_INVALID, "llama_generate: bad arguments");
    Model& m = *static_cast<Model*>(model);
    int32_t st[4];
    KVHP_HIP(hipMemcpyAsync(st, m.state, sizeof st, hipMemcpyDeviceToHost, m.stream),
             "hipMemcpyAsync(state)");
    KVHP_HIP(hipStreamSynchronize(m.stream), "hipStreamSynchronize");
    KVHP_REQUIRE(m.prompt_len > 0, KVHP_ERR_INVALID, "llama_generate: no prefill yet");
    KVHP_REQUIRE(st[0] + n_steps - 1 <= m.max_ctx, KVHP_ERR_INVALID,
                 "llama_generate: %d more tokens overflow the context of %d", n_steps,
                 m.max_ctx);
    if (use_graph && !m.graph_exec) {
        KVHP_HIP(hipStreamBeginCapture(m.stream, hipStreamCaptureModeThreadLocal),
                 "hipStreamBeginCapture");
        const int rc = decode_step_kernels(m, false);
        hipGraph_t g = nullptr;
        const hipError_t e = hipStreamEndCapture(m.stream, &g);
        if (rc) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        KVHP_HIP(e, "hipStreamEndCapture");
        m.graph = g;
        KVHP_HIP(hipGraphInstantiate(&m.graph_exec, m.graph, nullptr, nullptr, 0),
                 "hipGraphInstantiate");
    }
    hipEvent_t e0 = nullptr, e1 = nullptr;
    KVHP_HIP(hipEventCreate(&e0), "hipEventCreate");
    KVHP_HIP(hipEventCreate(&e1), "hipEventCreate");
    KVHP_HIP(hipEventRecord(e0, m.stream), "hipEventRecord");
    for (int i = 0; i < n_steps; ++i) {
        if (use_graph)
            KVHP_HIP(hipGraphLaunch(m.graph_exec, m.stream), "hipGraphLaunch");
        else
            KVHP_TRY(decode_step_kernels(m, false));
    }
    KVHP_HIP(hipEventRecord(e1, m.stream), "hipEventRecord");
    KVHP_HIP(hipEventSynchronize(e1), "hipEventSynchronize");
    float ms = 0.f;
    KVHP_HIP(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (elapsed_ms) *elapsed_ms = ms;
    if (tokens_out) {
        KVHP_HIP(hipMemcpyAsync(st, m.state, sizeof st, hipMemcpyDeviceToHost, m.stream),
                 "hipMemcpyAsync(state)");
        KVHP_HIP(hipStreamSynchronize(m.stream), "hipStreamSynchronize");
        // the log holds the prefill token then one token per decode step
        KVHP_HIP(hipMemcpy(tokens_out, m.log, (size_t)st[2] * 4, hipMemcpyDeviceToHost),
                 "hipMemcpy(log)");
    }
    return KVHP_OK;
}

extern "C" int kvhp_llama_tensor(void* model, int layer, int which, void** ptr, size_t* count) {
    clear_error();
    KVHP_REQUIRE(model && ptr && count, KVHP_ERR_INVALID, "llama_tensor: null argument");
    Model& m = *static_cast<Model*>(model);
    const kvhp_llama_config& c = m.c;
    const size_t H = c.hidden_size, D = c.head_dim, Hq = c.num_q_heads, Hkv = c.num_kv_heads;
    const size_t F = c.ffn_size, V = c.vocab_size;
    if (layer < 0) {
        switch (which) {
            case KVHP_LLAMA_EMBED: *ptr = m.embed; *count = V * H; return KVHP_OK;
            case KVHP_LLAMA_LM_HEAD: *ptr = m.lm_head; *count = V * H; return KVHP_OK;
            case KVHP_LLAMA_FINAL_NORM: *ptr = m.final_norm; *count = H; return KVHP_OK;
            default: break;
        }
    } else if (layer < c.num_layers) {
        const Layer& L = m.layers[layer];
        switch (which) {
            case KVHP_LLAMA_ATTN_NORM: *ptr = L.attn_norm; *count = H; return KVHP_OK;
            case KVHP_LLAMA_FFN_NORM: *ptr = L.ffn_norm; *count = H; return KVHP_OK;
            case KVHP_LLAMA_W_QKV: *ptr = L.w_qkv; *count = (Hq + 2 * Hkv) * D * H; return KVHP_OK;
            case KVHP_LLAMA_W_O: *ptr = L.w_o; *count = H * Hq * D; return KVHP_OK;
            case KVHP_LLAMA_W_GATE_UP: *ptr = L.w_gate_up; *count = 2 * F * H; return KVHP_OK;
            case KVHP_LLAMA_W_DOWN: *ptr = L.w_down; *count = H * F; return KVHP_OK;
            case KVHP_LLAMA_POOL_K: *ptr = L.pool_k; *count = Hkv * m.P * kPage * D; return KVHP_OK;
            case KVHP_LLAMA_POOL_V: *ptr = L.pool_v; *count = Hkv * m.P * kPage * D; return KVHP_OK;
            default: break;
        }
    }
    return fail(KVHP_ERR_INVALID, "llama_tensor: no tensor %d of layer %d", which, layer);
}
