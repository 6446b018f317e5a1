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
// Batched serving (kvhp_llama_prefill_paged / kvhp_llama_decode_paged) runs
// the same layers over a caller-owned page pool [L][2][Hkv][P][16][D] (the
// engine::PagedKVCache layout) and caller block tables, per the reference
// runner contract (docs/runner_interface.md:18-53): the caller has already
// allocated pages and bumped lengths; a decode step appends each sequence's
// K/V at its write position and attends over its seq_len keys; B sequences
// go through each projection as one B-row GEMM.
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

#include <algorithm>
#include <cstring>
#include <memory>
#include <vector>

namespace kvhp {
namespace {

constexpr float kInitStd = 0.02f;
constexpr int kShortSuffix = 32;  // cached-prefix suffixes up to this run as one batched step

struct Layer {
    f16* attn_norm = nullptr;  // [H]
    f16* ffn_norm = nullptr;   // [H]
    f16* w_qkv = nullptr;      // [(Hq + 2Hkv) D][H]
    f16* w_o = nullptr;        // [H][Hq D]
    f16* w_gate_up = nullptr;  // [2F][H]
    f16* w_down = nullptr;     // [H][F]
    // the four projections tiled for the batched kernels (kvhp_rows_tile_weights);
    // built on the first batched step, rebuilt by kvhp_llama_reserve
    f16 *w_qkv_t = nullptr, *w_o_t = nullptr, *w_gate_up_t = nullptr, *w_down_t = nullptr;
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
    f16* pool = nullptr;       // [L][2][Hkv][P][16][D], layer pools point into it
    int32_t* bt = nullptr;     // [P] identity page order
    // prefill activations, sized for max_ctx rows
    f16 *hidden = nullptr, *norm = nullptr, *qkv = nullptr, *q = nullptr, *k = nullptr,
        *v = nullptr, *attn = nullptr, *gu = nullptr, *act = nullptr;
    // decode activations
    f16 *x = nullptr, *q1 = nullptr, *attn1 = nullptr, *act1 = nullptr;
    float* logits = nullptr;   // [V]
    int32_t* tokens = nullptr; // [max_ctx] prompt ids
    int32_t* state = nullptr;  // [0] seq_len, [1] current token, [2] log count,
                               // [3] token of a paged prefill
    int32_t* log = nullptr;    // [max_ctx] generated tokens
    int32_t* aux = nullptr;    // cached-prefix prefill: replicated block-table rows, lengths
    size_t aux_words = 0;
    float* suffix_logits = nullptr;  // [kShortSuffix][V]: logits of a short cached-prefix prefill
    int32_t* suffix_next = nullptr;  // [kShortSuffix]
    void* ws = nullptr;        // decode attention workspace of the batch-1 step
    size_t ws_bytes = 0;
    void* ws_rows = nullptr;   // decode attention workspace of the batched paths (grows)
    size_t ws_rows_bytes = 0;
    void* part_rows = nullptr; // K-split partials of the batched down projection (grows)
    size_t part_rows_bytes = 0;
    int prompt_len = 0;
    bool rows_ok = false;      // batched projections fit the skinny-GEMM kernels
    f16* lm_head_t = nullptr;  // LM head tiled for the batched kernels
    bool tiled = false;        // the tiled copies hold the current weights
    // batched-step activations (2..32 rows), row-tiled (act_tiled_index):
    // hidden [32][H], attention output [32][Hq*D], SwiGLU output [32][F]
    f16 *hidden_t = nullptr, *attn_t = nullptr, *act_t = nullptr;
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

// Replace the model-owned buffer *p (of *cap elements) by one of at least n
// elements (twice the old size at least, so a model retires few buffers).
// The retired buffer stays allocated until kvhp_llama_destroy: a HIP graph
// that captured an earlier call keeps valid addresses, and nothing has to
// wait for the stream.  While `s` is capturing a graph nothing is allocated
// (the allocation cannot be captured): KVHP_ERR_WORKSPACE, so size the
// buffers first with kvhp_llama_reserve (or one eager call of the largest
// shape).  On failure *p and *cap are unchanged.
template <typename T>
int regrow(Model& m, T** p, size_t* cap, size_t n, hipStream_t s, const char* what) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    KVHP_HIP(hipStreamIsCapturing(s, &st), "hipStreamIsCapturing(regrow)");
    KVHP_REQUIRE(st == hipStreamCaptureStatusNone, KVHP_ERR_WORKSPACE,
                 "%s: the model's buffer must grow from %zu to %zu elements, which cannot happen "
                 "under graph capture (call kvhp_llama_reserve before capturing)",
                 what, *cap, n);
    if (n < 2 * *cap) n = 2 * *cap;
    T* fresh = nullptr;
    KVHP_TRY(alloc_n(m, n, &fresh));
    *p = fresh;
    *cap = n;
    return KVHP_OK;
}

// Decode-attention workspace for B sequences of up to max_seq_len keys,
// owned by the model (not the library's per-device buffer), so that models
// on different streams never share split partials.
int rows_workspace(Model& m, int B, int max_seq_len, hipStream_t s, void** ws, size_t* bytes) {
    const kvhp_llama_config& c = m.c;
    const size_t need = kvhp_decode_workspace_bytes(B, c.num_q_heads, c.num_kv_heads, c.head_dim,
                                                    max_seq_len, 0);
    if (need > m.ws_rows_bytes) {
        char* p = static_cast<char*>(m.ws_rows);
        KVHP_TRY(regrow(m, &p, &m.ws_rows_bytes, need, s, "decode-attention workspace"));
        m.ws_rows = p;
    }
    *ws = m.ws_rows;
    *bytes = m.ws_rows_bytes;
    return KVHP_OK;
}

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

// C[M][N] = A[M][K] W[N][K]^T with fp32 C (the batched LM head).
int linear_f32(Model& m, const f16* A, const f16* W, float* C, int M, int N, int K) {
    const float alpha = 1.f, beta = 0.f;
    return blas_check(rocblas_gemm_ex(m.blas, rocblas_operation_transpose,
                                      rocblas_operation_none, N, M, K, &alpha, W,
                                      rocblas_datatype_f16_r, K, A, rocblas_datatype_f16_r, K,
                                      &beta, C, rocblas_datatype_f32_r, N, C,
                                      rocblas_datatype_f32_r, N, rocblas_datatype_f32_r,
                                      rocblas_gemm_algo_standard, 0, 0),
                      "linear_f32");
}

// K/V pages a forward writes and reads: pool [L][2][Hkv][num_pages][16][D]
// and block-table rows of max_pages entries.
struct Pages {
    f16* base;
    int num_pages;
    const int32_t* bt;
    int max_pages;
};

f16* layer_pool(const Model& m, const Pages& pg, int l, int is_v) {
    return pg.base + (size_t)(2 * l + is_v) * m.c.num_kv_heads * pg.num_pages * kPage * m.c.head_dim;
}

kvhp_kv_view pages_view(const Model& m, const Pages& pg, int l, int is_v) {
    kvhp_kv_view v{};
    v.data = layer_pool(m, pg, l, is_v);
    v.stride_b = 0;
    v.stride_h = (int64_t)pg.num_pages * kPage * m.c.head_dim;
    v.stride_s = m.c.head_dim;
    v.stride_d = 1;
    v.block_table = pg.bt;
    v.max_pages = pg.max_pages;
    v.page_size = kPage;
    v.num_pages = pg.num_pages;
    return v;
}

Pages own_pages(const Model& m) { return Pages{m.pool, m.P, m.bt, m.P}; }

// The model's own pages are in identity order, so its pool [Hkv][P][16][D]
// is the contiguous cache [Hkv][16 P][D]: the batch-1 step reads it through
// a strided view, with no block-table load ahead of the first K/V load.
kvhp_kv_view own_view(const Model& m, int l, int is_v) {
    kvhp_kv_view v{};
    v.data = layer_pool(m, own_pages(m), l, is_v);
    v.stride_b = 0;
    v.stride_h = (int64_t)m.P * kPage * m.c.head_dim;
    v.stride_s = m.c.head_dim;
    v.stride_d = 1;
    return v;
}

// rocBLAS follows `s` for the lifetime of this object, then the model's
// stream again.
struct BlasOn {
    Model& m;
    BlasOn(Model& mm, hipStream_t s) : m(mm) { (void)rocblas_set_stream(m.blas, s); }
    ~BlasOn() { (void)rocblas_set_stream(m.blas, m.stream); }
};

// Prompt forward of m.tokens[0, n) (one sequence): final hidden rows in
// m.hidden, the K/V of every position written through pg.bt (ids -1, pages
// held by other sequences, are skipped by the writes).
int prefill_layers(Model& m, int n, const Pages& pg, void* s) {
    const kvhp_llama_config& c = m.c;
    const int H = c.hidden_size, D = c.head_dim, Hq = c.num_q_heads, Hkv = c.num_kv_heads;
    const int F = c.ffn_size, NQKV = (Hq + 2 * Hkv) * D;
    KVHP_TRY(kvhp_embedding(m.tokens, m.embed, m.hidden, n, H, c.vocab_size, s));
    for (int l = 0; l < c.num_layers; ++l) {
        const Layer& L = m.layers[l];
        KVHP_TRY(kvhp_rmsnorm(m.hidden, L.attn_norm, m.norm, n, H, c.rms_eps, s));
        KVHP_TRY(linear(m, m.norm, L.w_qkv, m.qkv, n, NQKV, H, false));
        KVHP_TRY(kvhp_split_qkv_rope(m.qkv, n, Hq, Hkv, D, 0, c.rope_theta, m.q, m.k, m.v, s));
        KVHP_TRY(kvhp_flash_prefill_paged(m.q, m.k, m.v, m.attn, n, Hq, Hkv, D, 1,
                                          layer_pool(m, pg, l, 0), layer_pool(m, pg, l, 1), pg.bt,
                                          pg.max_pages, pg.num_pages, s));
        KVHP_TRY(linear(m, m.attn, L.w_o, m.hidden, n, H, Hq * D, true));
        KVHP_TRY(kvhp_rmsnorm(m.hidden, L.ffn_norm, m.norm, n, H, c.rms_eps, s));
        KVHP_TRY(linear(m, m.norm, L.w_gate_up, m.gu, n, 2 * F, H, false));
        KVHP_TRY(kvhp_swiglu_rows(m.gu, m.act, n, F, s));
        KVHP_TRY(linear(m, m.act, L.w_down, m.hidden, n, H, F, true));
    }
    return KVHP_OK;
}

// Inputs of a cached-prefix prefill's attention, on the device: row r of
// tables [rows][width] is the sequence's block-table row, lens[r] =
// first + r + 1 (query row r sits at position first + r), start[0] = first.
__global__ void suffix_rows_kernel(int32_t* tables, int32_t* wtables, int32_t* lens,
                                   int32_t* pos, int32_t* start, const int32_t* row,
                                   const int32_t* wrow, int rows, int width, int first) {
    const int64_t total = (int64_t)rows * width;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        tables[i] = row[i % width];
        wtables[i] = wrow[i % width];
    }
    for (int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; r < rows;
         r += (int64_t)gridDim.x * blockDim.x) {
        lens[r] = first + static_cast<int32_t>(r) + 1;
        pos[r] = first + static_cast<int32_t>(r);
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) start[0] = first;
}

// Device inputs of a cached-prefix prefill of `rows` suffix rows (in m.aux):
// replicated read and write block-table rows, lengths, positions, start.
struct SuffixRows {
    int32_t *tables, *wtables, *lens, *pos, *start;
};

int suffix_rows(Model& m, const Pages& pg, const int32_t* write_bt, int first, int rows,
                hipStream_t s, SuffixRows& out) {
    const size_t words = 2 * (size_t)rows * pg.max_pages + 2 * (size_t)rows + 1;
    if (m.aux_words < words)
        KVHP_TRY(regrow(m, &m.aux, &m.aux_words, words, s, "suffix block tables"));
    out.tables = m.aux;
    out.wtables = out.tables + (size_t)rows * pg.max_pages;
    out.lens = out.wtables + (size_t)rows * pg.max_pages;
    out.pos = out.lens + rows;
    out.start = out.pos + rows;
    const int64_t blocks = std::min<int64_t>(((int64_t)rows * pg.max_pages + 255) / 256, 1024);
    hipLaunchKernelGGL(suffix_rows_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s,
                       out.tables, out.wtables, out.lens, out.pos, out.start, pg.bt, write_bt,
                       rows, pg.max_pages, first);
    return check_launch("suffix_rows");
}

// "Full" prefix mode: only prompt positions [first, n) run through the
// model (m.tokens holds all n ids).  Their K/V are appended through
// write_bt (the block-table row, or it with shared pages set to -1), and
// query row r attends over keys
// [0, first + r + 1) from the pages -- the cached prefix included -- as one
// row of a batched decode-attention call.  Final hidden rows in m.hidden.
int prefill_suffix_layers(Model& m, int first, int n, const Pages& pg, const int32_t* write_bt,
                          hipStream_t s) {
    const kvhp_llama_config& c = m.c;
    const int H = c.hidden_size, D = c.head_dim, Hq = c.num_q_heads, Hkv = c.num_kv_heads;
    const int F = c.ffn_size, NQKV = (Hq + 2 * Hkv) * D;
    const int S = n - first;
    SuffixRows sr{};
    KVHP_TRY(suffix_rows(m, pg, write_bt, first, S, s, sr));
    int32_t* lens = sr.lens;
    int32_t* start = sr.start;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    KVHP_TRY(rows_workspace(m, S, n, s, &ws, &ws_bytes));
    const Pages rows_pg{pg.base, pg.num_pages, sr.tables, pg.max_pages};
    KVHP_TRY(kvhp_embedding(m.tokens + first, m.embed, m.hidden, S, H, c.vocab_size, s));
    for (int l = 0; l < c.num_layers; ++l) {
        const Layer& L = m.layers[l];
        KVHP_TRY(kvhp_rmsnorm(m.hidden, L.attn_norm, m.norm, S, H, c.rms_eps, s));
        KVHP_TRY(linear(m, m.norm, L.w_qkv, m.qkv, S, NQKV, H, false));
        KVHP_TRY(kvhp_split_qkv_rope(m.qkv, S, Hq, Hkv, D, first, c.rope_theta, m.q, m.k, m.v, s));
        KVHP_TRY(kvhp_paged_append_kv(m.k, m.v, layer_pool(m, pg, l, 0), layer_pool(m, pg, l, 1),
                                      write_bt, pg.max_pages, start, 1, S, Hkv, D, pg.num_pages,
                                      s));
        const kvhp_kv_view kv = pages_view(m, rows_pg, l, 0), vv = pages_view(m, rows_pg, l, 1);
        KVHP_TRY(kvhp_decode_attention(m.q, &kv, &vv, lens, m.attn, S, Hq, Hkv, D, n, 0, ws,
                                       ws_bytes, s));
        KVHP_TRY(linear(m, m.attn, L.w_o, m.hidden, S, H, Hq * D, true));
        KVHP_TRY(kvhp_rmsnorm(m.hidden, L.ffn_norm, m.norm, S, H, c.rms_eps, s));
        KVHP_TRY(linear(m, m.norm, L.w_gate_up, m.gu, S, 2 * F, H, false));
        KVHP_TRY(kvhp_swiglu_rows(m.gu, m.act, S, F, s));
        KVHP_TRY(linear(m, m.act, L.w_down, m.hidden, S, H, F, true));
    }
    return KVHP_OK;
}

// One batched decode step: row b takes token tokens[b] at position
// positions[b] (its K/V appended there through row b of pg.bt) and attends
// over seq_lens[b] keys; fp32 logits [B][V], greedy tokens next[b].  One row
// runs on the batch-1 step's GEMV kernels, up to 32 on the fused skinny-GEMM
// kernels, larger batches on library GEMMs with separate RMSNorm / RoPE /
// SwiGLU launches.
// Tiled copies of the projection weights for the batched kernels (each weight
// load 1 KB contiguous; bit-identical outputs): allocated once, (re)written
// from the row-major weights on stream s.  Not under graph capture (an
// allocation and copies a replay must not repeat): kvhp_llama_reserve builds
// them before.
int build_tiled(Model& m, hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    KVHP_HIP(hipStreamIsCapturing(s, &st), "hipStreamIsCapturing(tiled weights)");
    KVHP_REQUIRE(st == hipStreamCaptureStatusNone, KVHP_ERR_WORKSPACE,
                 "decode_paged: the batched projections' tiled weights are built on the first "
                 "batched step, which cannot happen under graph capture (call "
                 "kvhp_llama_reserve before capturing)");
    const kvhp_llama_config& c = m.c;
    const int H = c.hidden_size, D = c.head_dim, Hq = c.num_q_heads, Hkv = c.num_kv_heads;
    const int F = c.ffn_size;
    auto tile = [&](f16** dst, int kind, const f16* W, int N, int K) {
        if (!*dst) {
            const size_t nb = kvhp_rows_tiled_bytes(kind, N, K, Hq, Hkv, D);
            KVHP_REQUIRE(nb > 0, KVHP_ERR_UNSUPPORTED, "tiled weights: %d x %d", N, K);
            KVHP_TRY(alloc_n(m, nb / sizeof(f16), dst));
        }
        return kvhp_rows_tile_weights(kind, W, N, K, Hq, Hkv, D, *dst, s);
    };
    for (Layer& L : m.layers) {
        KVHP_TRY(tile(&L.w_qkv_t, KVHP_ROWS_QKV, L.w_qkv, 0, H));
        KVHP_TRY(tile(&L.w_o_t, KVHP_ROWS_PLAIN, L.w_o, H, Hq * D));
        KVHP_TRY(tile(&L.w_gate_up_t, KVHP_ROWS_SWIGLU, L.w_gate_up, F, H));
        KVHP_TRY(tile(&L.w_down_t, KVHP_ROWS_PLAIN, L.w_down, H, F));
    }
    KVHP_TRY(tile(&m.lm_head_t, KVHP_ROWS_PLAIN, m.lm_head, c.vocab_size, H));
    if (!m.hidden_t) {
        KVHP_TRY(alloc_n(m, (size_t)32 * H, &m.hidden_t));
        KVHP_TRY(alloc_n(m, (size_t)32 * Hq * D, &m.attn_t));
        KVHP_TRY(alloc_n(m, (size_t)32 * F, &m.act_t));
    }
    m.tiled = true;
    return KVHP_OK;
}

int decode_rows(Model& m, const int32_t* tokens, int B, const Pages& pg,
                const int32_t* positions, const int32_t* seq_lens, int max_seq_len,
                float* logits, int32_t* next, void* s, const int32_t* write_bt = nullptr) {
    // K/V appends go through write_bt when given (rows [B][max_pages] with
    // shared pages -1), reads through pg.bt; only the fused paths (one row,
    // or up to 32 on the batched projections) take it
    KVHP_REQUIRE(write_bt == nullptr || B == 1 || (B <= 32 && m.rows_ok), KVHP_ERR_INVALID,
                 "decode_rows: a separate write table needs the fused projections");
    const int32_t* wbt = write_bt ? write_bt : pg.bt;
    const kvhp_llama_config& c = m.c;
    const int H = c.hidden_size, D = c.head_dim, Hq = c.num_q_heads, Hkv = c.num_kv_heads;
    const int F = c.ffn_size, NQKV = (Hq + 2 * Hkv) * D;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    KVHP_TRY(rows_workspace(m, B, max_seq_len, static_cast<hipStream_t>(s), &ws, &ws_bytes));
    if (B > 1 && B <= 32 && m.rows_ok && !m.tiled)
        KVHP_TRY(build_tiled(m, static_cast<hipStream_t>(s)));
    if (B == 1 || B > 32 || !m.rows_ok)
        KVHP_TRY(kvhp_embedding(tokens, m.embed, m.hidden, B, H, c.vocab_size, s));
    if (B == 1) {
        // one sequence: the batch-1 step's GEMV kernels (no padded MFMA columns)
        for (int l = 0; l < c.num_layers; ++l) {
            const Layer& L = m.layers[l];
            KVHP_TRY(rmsnorm_qkv_rope_append_at(L.w_qkv, m.hidden, L.attn_norm, c.rms_eps,
                                                positions, c.rope_theta, m.q,
                                                layer_pool(m, pg, l, 0), layer_pool(m, pg, l, 1),
                                                wbt, pg.max_pages, pg.num_pages, Hq, Hkv, D, H,
                                                static_cast<hipStream_t>(s)));
            const kvhp_kv_view kv = pages_view(m, pg, l, 0), vv = pages_view(m, pg, l, 1);
            KVHP_TRY(kvhp_decode_attention(m.q, &kv, &vv, seq_lens, m.attn, 1, Hq, Hkv, D,
                                           max_seq_len, 0, ws, ws_bytes, s));
            KVHP_TRY(kvhp_gemv_residual(L.w_o, m.attn, m.hidden, m.hidden, H, Hq * D, s));
            KVHP_TRY(kvhp_rmsnorm_gemv_swiglu(L.w_gate_up, m.hidden, L.ffn_norm, c.rms_eps, m.act,
                                              F, H, s));
            KVHP_TRY(kvhp_gemv_residual(L.w_down, m.act, m.hidden, m.hidden, H, F, s));
        }
        KVHP_TRY(kvhp_rmsnorm_gemv(m.lm_head, m.hidden, m.final_norm, c.rms_eps, nullptr, logits,
                                   c.vocab_size, H, s));
        return kvhp_argmax_rows(logits, 1, c.vocab_size, next, s);
    }
    if (B <= 32 && m.rows_ok) {
        // Skinny-GEMM projections with the batch-1 step's fusions: every
        // weight read once per step for all B rows, from its tiled copy, six
        // launches per layer (seven when the down projection's x is large
        // enough to split over K: its partials live in the model's own
        // buffer).  The activations between them (hidden state, attention
        // output, SwiGLU output) stay row-tiled, so every projection loads
        // its x as 1 KB contiguous per wave and k step (bit-identical to
        // row-major activations: the same operands).
        const int nt = act_tiles_for(B);
        const hipStream_t hs = static_cast<hipStream_t>(s);
        const size_t part_need = kvhp_gemv_rows_workspace_bytes(H, F, B);
        if (part_need > m.part_rows_bytes) {
            char* p = static_cast<char*>(m.part_rows);
            KVHP_TRY(regrow(m, &p, &m.part_rows_bytes, part_need, static_cast<hipStream_t>(s),
                            "down-projection partials"));
            m.part_rows = p;
        }
        KVHP_TRY(embedding_act(tokens, m.embed, m.hidden_t, B, H, c.vocab_size, nt, hs));
        for (int l = 0; l < c.num_layers; ++l) {
            const Layer& L = m.layers[l];
            KVHP_TRY(qkv_rows_act(L.w_qkv_t, m.hidden_t, L.attn_norm, c.rms_eps, positions,
                                  c.rope_theta, m.q, layer_pool(m, pg, l, 0),
                                  layer_pool(m, pg, l, 1), wbt, pg.max_pages, pg.num_pages, Hq,
                                  Hkv, D, H, B, nt, hs));
            const kvhp_kv_view kv = pages_view(m, pg, l, 0), vv = pages_view(m, pg, l, 1);
            KVHP_TRY(decode_attention_act(m.q, &kv, &vv, seq_lens, m.attn_t, B, Hq, Hkv, D,
                                          max_seq_len, ws, ws_bytes, nt, hs));
            KVHP_TRY(residual_rows_act(L.w_o_t, m.attn_t, m.hidden_t, m.hidden_t, H, Hq * D, B,
                                       nullptr, 0, nt, nt, hs));
            KVHP_TRY(swiglu_rows_act(L.w_gate_up_t, m.hidden_t, L.ffn_norm, c.rms_eps, m.act_t,
                                     F, H, B, nt, hs));
            KVHP_TRY(residual_rows_act(L.w_down_t, m.act_t, m.hidden_t, m.hidden_t, H, F, B,
                                       part_need ? m.part_rows : nullptr, part_need, nt, nt, hs));
        }
        KVHP_TRY(rmsnorm_rows_act(m.lm_head_t, m.hidden_t, m.final_norm, c.rms_eps, nullptr,
                                  logits, c.vocab_size, H, B, nt, hs));
        return kvhp_argmax_rows(logits, B, c.vocab_size, next, s);
    }
    for (int l = 0; l < c.num_layers; ++l) {
        const Layer& L = m.layers[l];
        KVHP_TRY(kvhp_rmsnorm(m.hidden, L.attn_norm, m.norm, B, H, c.rms_eps, s));
        KVHP_TRY(linear(m, m.norm, L.w_qkv, m.qkv, B, NQKV, H, false));
        KVHP_TRY(kvhp_split_qkv_rope_rows(m.qkv, B, Hq, Hkv, D, positions, c.rope_theta, m.q, m.k,
                                          m.v, s));
        const kvhp_kv_view kv = pages_view(m, pg, l, 0), vv = pages_view(m, pg, l, 1);
        KVHP_TRY(kvhp_paged_append_decode(m.q, m.k, m.v, &kv, &vv, positions, seq_lens, m.attn, B,
                                          Hq, Hkv, D, max_seq_len, 0, ws, ws_bytes, s));
        KVHP_TRY(linear(m, m.attn, L.w_o, m.hidden, B, H, Hq * D, true));
        KVHP_TRY(kvhp_rmsnorm(m.hidden, L.ffn_norm, m.norm, B, H, c.rms_eps, s));
        KVHP_TRY(linear(m, m.norm, L.w_gate_up, m.gu, B, 2 * F, H, false));
        KVHP_TRY(kvhp_swiglu_rows(m.gu, m.act, B, F, s));
        KVHP_TRY(linear(m, m.act, L.w_down, m.hidden, B, H, F, true));
    }
    KVHP_TRY(kvhp_rmsnorm(m.hidden, m.final_norm, m.norm, B, H, c.rms_eps, s));
    KVHP_TRY(linear_f32(m, m.norm, m.lm_head, logits, B, c.vocab_size, H));
    return kvhp_argmax_rows(logits, B, c.vocab_size, next, s);
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
        const int l = static_cast<int>(&L - m.layers.data());
        const kvhp_kv_view kv = own_view(m, l, 0), vv = own_view(m, l, 1);
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
    // the model's own pages: one block [L][2][Hkv][P][16][D], the layout of a
    // caller-owned pool (engine::PagedKVCache)
    const size_t pool = (size_t)Hkv * m->P * kPage * D;
    KVHP_TRY(alloc_n(*m, pool * 2 * c.num_layers, &m->pool));
    KVHP_HIP(hipMemsetAsync(m->pool, 0, pool * 2 * c.num_layers * 2, m->stream),
             "hipMemsetAsync(pool)");
    for (int l = 0; l < c.num_layers; ++l) {
        Layer& L = m->layers[l];
        KVHP_TRY(ones(&L.attn_norm, H));
        KVHP_TRY(ones(&L.ffn_norm, H));
        KVHP_TRY(randn(&L.w_qkv, (size_t)NQKV * H));
        KVHP_TRY(randn(&L.w_o, (size_t)H * Hq * D));
        KVHP_TRY(randn(&L.w_gate_up, (size_t)2 * F * H));
        KVHP_TRY(randn(&L.w_down, (size_t)H * F));
        L.pool_k = m->pool + (size_t)(2 * l) * pool;
        L.pool_v = m->pool + (size_t)(2 * l + 1) * pool;
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
    KVHP_TRY(alloc_n(*m, (size_t)kShortSuffix * V, &m->suffix_logits));
    KVHP_TRY(alloc_n(*m, kShortSuffix, &m->suffix_next));
    // K = hidden (q/k/v, gate/up, LM head), Hq*D (o) and ffn (down): 256*n
    // with n <= 8, or 352*n with n <= 16 for the down projection
    auto k256 = [](int K) { return K % 256 == 0 && K / 256 <= 8; };
    m->rows_ok = k256(H) && (k256(F) || (F % 352 == 0 && F / 352 <= 16)) && D % 32 == 0;
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
    const int H = c.hidden_size;
    void* s = m.stream;
    KVHP_HIP(hipMemcpyAsync(m.tokens, tokens, (size_t)n * 4, hipMemcpyHostToDevice, m.stream),
             "hipMemcpyAsync(tokens)");
    // state: seq_len = n (bumped to n+1 by the argmax), log count 0
    const int32_t st[4] = {n, 0, 0, 0};
    KVHP_HIP(hipMemcpyAsync(m.state, st, sizeof st, hipMemcpyHostToDevice, m.stream),
             "hipMemcpyAsync(state)");
    KVHP_TRY(prefill_layers(m, n, own_pages(m), s));
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

namespace {
// Prefill over caller pages: positions [first, n) of the n prompt ids run
// through the model (first = 0: the whole prompt by the flash prefill
// kernel; first > 0: the suffix attends the cached prefix from the pages);
// logits and greedy token of the last position.
int prefill_pages(void* model, const int32_t* tokens, int n, int first, void* pool, int num_pages,
                  const int32_t* block_table, const int32_t* write_table, int max_pages,
                  float* logits_out, int32_t* next_token, void* stream, const char* what) {
    KVHP_REQUIRE(model && tokens && n > 0 && pool && block_table && num_pages > 0 &&
                     max_pages > 0,
                 KVHP_ERR_INVALID, "%s: bad arguments", what);
    KVHP_REQUIRE(first >= 0 && first < n, KVHP_ERR_INVALID,
                 "%s: %d cached tokens of a %d-token prompt", what, first, n);
    Model& m = *static_cast<Model*>(model);
    const kvhp_llama_config& c = m.c;
    KVHP_REQUIRE(n <= m.max_ctx, KVHP_ERR_INVALID,
                 "%s: %d tokens exceed the model's %d activation rows", what, n, m.max_ctx);
    KVHP_REQUIRE((int64_t)n <= (int64_t)max_pages * kPage, KVHP_ERR_INVALID,
                 "%s: %d tokens exceed %d pages", what, n, max_pages);
    hipStream_t s = static_cast<hipStream_t>(stream);
    BlasOn on(m, s);
    const Pages pg{static_cast<f16*>(pool), num_pages, block_table, max_pages};
    KVHP_HIP(hipMemcpyAsync(m.tokens, tokens, (size_t)n * 4, hipMemcpyHostToDevice, s),
             "hipMemcpyAsync(tokens)");
    const int S = n - first;
    const float* last_logits = m.logits;
    const int32_t* last_tok = m.state + 3;
    if (first > 0 && S <= kShortSuffix && (S == 1 || m.rows_ok)) {
        // a short suffix is one batched decode step: row r at position
        // first + r appends its K/V, then attends over first + r + 1 keys
        SuffixRows sr{};
        KVHP_TRY(suffix_rows(m, pg, write_table ? write_table : block_table, first, S, s, sr));
        const Pages rows_pg{pg.base, pg.num_pages, sr.tables, pg.max_pages};
        KVHP_TRY(decode_rows(m, m.tokens + first, S, rows_pg, sr.pos, sr.lens, n,
                             m.suffix_logits, m.suffix_next, s, sr.wtables));
        last_logits = m.suffix_logits + (size_t)(S - 1) * c.vocab_size;
        last_tok = m.suffix_next + S - 1;
    } else {
        if (first == 0)
            KVHP_TRY(prefill_layers(m, n, pg, s));
        else
            KVHP_TRY(prefill_suffix_layers(m, first, n, pg,
                                           write_table ? write_table : block_table, s));
        const int H = c.hidden_size;
        KVHP_TRY(kvhp_rmsnorm_gemv(m.lm_head, m.hidden + (size_t)(S - 1) * H, m.final_norm,
                                   c.rms_eps, nullptr, m.logits, c.vocab_size, H, s));
        KVHP_TRY(kvhp_argmax_rows(m.logits, 1, c.vocab_size, m.state + 3, s));
    }
    if (logits_out)
        KVHP_HIP(hipMemcpyAsync(logits_out, last_logits, (size_t)c.vocab_size * 4,
                                hipMemcpyDeviceToHost, s),
                 "hipMemcpyAsync(logits)");
    int32_t tok = 0;
    KVHP_HIP(hipMemcpyAsync(&tok, last_tok, 4, hipMemcpyDeviceToHost, s),
             "hipMemcpyAsync(token)");
    KVHP_HIP(hipStreamSynchronize(s), "hipStreamSynchronize(prefill)");
    if (next_token) *next_token = tok;
    return KVHP_OK;
}
}  // namespace

extern "C" int kvhp_llama_prefill_paged(void* model, const int32_t* tokens, int n, void* pool,
                                        int num_pages, const int32_t* block_table, int max_pages,
                                        float* logits_out, int32_t* next_token, void* stream) {
    clear_error();
    return prefill_pages(model, tokens, n, 0, pool, num_pages, block_table, nullptr, max_pages,
                         logits_out, next_token, stream, "llama_prefill_paged");
}

extern "C" int kvhp_llama_prefill_cached(void* model, const int32_t* tokens, int n,
                                         int num_cached, void* pool, int num_pages,
                                         const int32_t* block_table,
                                         const int32_t* write_table, int max_pages,
                                         float* logits_out, int32_t* next_token, void* stream) {
    clear_error();
    KVHP_REQUIRE(num_cached > 0, KVHP_ERR_INVALID,
                 "llama_prefill_cached: no cached tokens (kvhp_llama_prefill_paged runs the "
                 "whole prompt)");
    return prefill_pages(model, tokens, n, num_cached, pool, num_pages, block_table, write_table,
                         max_pages, logits_out, next_token, stream, "llama_prefill_cached");
}

extern "C" int kvhp_llama_decode_paged(void* model, const int32_t* tokens, int batch, void* pool,
                                       int num_pages, const int32_t* block_tables, int max_pages,
                                       const int32_t* positions, const int32_t* seq_lens,
                                       int max_seq_len, float* logits, int32_t* next_tokens,
                                       void* stream) {
    clear_error();
    KVHP_REQUIRE(model && tokens && pool && block_tables && positions && seq_lens && logits &&
                     next_tokens && num_pages > 0 && max_pages > 0 && max_seq_len > 0,
                 KVHP_ERR_INVALID, "llama_decode_paged: bad arguments");
    Model& m = *static_cast<Model*>(model);
    if (batch == 0) return KVHP_OK;
    KVHP_REQUIRE(batch > 0 && batch <= m.max_ctx, KVHP_ERR_INVALID,
                 "llama_decode_paged: batch %d outside 1..%d", batch, m.max_ctx);
    hipStream_t s = static_cast<hipStream_t>(stream);
    BlasOn on(m, s);
    const Pages pg{static_cast<f16*>(pool), num_pages, block_tables, max_pages};
    return decode_rows(m, tokens, batch, pg, positions, seq_lens, max_seq_len, logits, next_tokens,
                       s);
}

extern "C" int kvhp_llama_reserve(void* model, int max_batch, int max_seq_len) {
    clear_error();
    KVHP_REQUIRE(model && max_batch > 0 && max_seq_len > 0, KVHP_ERR_INVALID,
                 "llama_reserve: bad arguments");
    Model& m = *static_cast<Model*>(model);
    KVHP_REQUIRE(max_batch <= m.max_ctx, KVHP_ERR_INVALID,
                 "llama_reserve: batch %d outside 1..%d", max_batch, m.max_ctx);
    const kvhp_llama_config& c = m.c;
    // The auto split plan depends on both the batch and the longest length,
    // not monotonically (a grid cap per batch): take the largest workspace
    // over every batch and every length up to the limits (lengths in 64-key
    // steps, where the plan's chunk rounding changes, plus the limit itself).
    size_t ws_need = 0, part_need = 0;
    for (int b = 1; b <= max_batch; ++b) {
        for (int len = 64;; len += 64) {
            const int l = len < max_seq_len ? len : max_seq_len;
            const size_t w = kvhp_decode_workspace_bytes(b, c.num_q_heads, c.num_kv_heads,
                                                         c.head_dim, l, 0);
            if (w > ws_need) ws_need = w;
            if (l == max_seq_len) break;
        }
        if (b <= 32 && m.rows_ok) {
            const size_t pn = kvhp_gemv_rows_workspace_bytes(c.hidden_size, c.ffn_size, b);
            if (pn > part_need) part_need = pn;
        }
    }
    if (ws_need > m.ws_rows_bytes) {
        char* p = static_cast<char*>(m.ws_rows);
        KVHP_TRY(regrow(m, &p, &m.ws_rows_bytes, ws_need, nullptr, "llama_reserve"));
        m.ws_rows = p;
    }
    if (part_need > m.part_rows_bytes) {
        char* p = static_cast<char*>(m.part_rows);
        KVHP_TRY(regrow(m, &p, &m.part_rows_bytes, part_need, nullptr, "llama_reserve"));
        m.part_rows = p;
    }
    if (max_batch > 1 && m.rows_ok) {
        // the batched projections' tiled weights, from the weights as they
        // are now
        KVHP_TRY(build_tiled(m, m.stream));
        KVHP_HIP(hipStreamSynchronize(m.stream), "hipStreamSynchronize(llama_reserve)");
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
