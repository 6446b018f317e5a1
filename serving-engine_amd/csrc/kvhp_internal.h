// kvhp_internal.h -- shared definitions of the gfx950 KV-cache hot-path library.
//
// Device side: 16-bit float vector types, 16-byte load/store helpers, wave64
// DPP reductions.  Host side: thread-local error reporting and HIP error
// plumbing for the C ABI in include/kvhp_c.h.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "kvhp_c.h"

namespace kvhp {

typedef _Float16 f16;
typedef f16 half8 __attribute__((ext_vector_type(8)));
typedef f16 half4 __attribute__((ext_vector_type(4)));
typedef f16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kPage = KVHP_PAGE_SIZE;

// ---------------------------------------------------------------- host ----
void set_error(const char* fmt, ...);
void clear_error();
int fail(int code, const char* fmt, ...);
// Report the launch status of the kernels just enqueued.
int check_launch(const char* what);

// kvhp_argmax that also copies row `token` of embed [V][hidden] into x
// (model_ops.hip; used by the model runner so that a decode step starts
// from x without an embedding launch).
int argmax_embed(const float* logits, int64_t n, int32_t* token, int32_t* seq_len, int32_t* log,
                 int32_t* log_count, const void* embed, int64_t hidden, void* x, hipStream_t s);

// kvhp_rmsnorm_qkv_rope_append for one token at position *position (device
// int32; negative: nothing appended) rather than at seq_len[0] - 1
// (model_ops.hip; the batched runner's one-sequence step).
int rmsnorm_qkv_rope_append_at(const void* W_qkv, const void* x, const void* norm_w, float eps,
                               const int32_t* position, float rope_theta, void* q_out,
                               void* pool_k, void* pool_v, const int32_t* block_table,
                               int max_pages, int num_pages, int num_q_heads, int num_kv_heads,
                               int head_dim, int K, hipStream_t stream);

// Row-tiled activations: the batched runner keeps its hidden state, attention
// output and SwiGLU output ([B][K], K % 32 == 0) in the lane order of the 16x16x32 MFMA
// B operand, so that the batched projections load one k step of 16 batch
// rows as 1 KB contiguous per wave instead of staging row-major rows through
// LDS.  Element (b, k) sits at act_tiled_index(b, k,
// nbt), nbt = ceil(B / 16) batch tiles: 1 KB block (k / 32, b / 16), lane
// 16 (k % 32 / 8) + b % 16, element k % 8.  Eight consecutive k from a
// multiple of 8 stay contiguous.  Rows past B inside the last tile are
// padding (never read into a kept result).
__host__ __device__ __forceinline__ int64_t act_tiled_index(int64_t b, int64_t k, int nbt) {
    return ((((k >> 5) * nbt + (b >> 4)) * 64 + 16 * ((k & 31) >> 3) + (b & 15)) << 3) +
           (k & 7);
}
inline int act_tiles_for(int batch) { return (batch + 15) / 16; }

// The batched runner's entry points on row-tiled activations (act_tiles =
// act_tiles_for(batch); 0: row-major, as the exported kvhp_* functions), in
// model_ops.hip: the same kernels as kvhp_gemv_residual_rows_tiled /
// kvhp_rmsnorm_gemv_rows_tiled / kvhp_rmsnorm_gemv_swiglu_rows_tiled /
// kvhp_rmsnorm_qkv_rope_append_rows_tiled and kvhp_embedding, with x, the
// residual and fp16 outputs in that layout (q, the pages and fp32 logits stay
// as they are).  The residual projection takes the layouts of x and of the
// residual stream separately.
int residual_rows_act(const void* Wt, const void* x, const void* r, void* y, int N, int K,
                      int batch, void* workspace, size_t workspace_bytes, int x_tiles,
                      int y_tiles, hipStream_t s);
int rmsnorm_rows_act(const void* Wt, const void* x, const void* norm_w, float eps, void* y16,
                     float* y32, int N, int K, int batch, int act_tiles, hipStream_t s);
int swiglu_rows_act(const void* Wt, const void* x, const void* norm_w, float eps, void* out,
                    int N, int K, int batch, int act_tiles, hipStream_t s);
int qkv_rows_act(const void* Wt, const void* x, const void* norm_w, float eps,
                 const int32_t* positions, float rope_theta, void* q_out, void* pool_k,
                 void* pool_v, const int32_t* block_tables, int max_pages, int num_pages,
                 int num_q_heads, int num_kv_heads, int head_dim, int K, int batch, int act_tiles,
                 hipStream_t s);
int embedding_act(const int32_t* token_ids, const void* table, void* out, int batch,
                  int64_t hidden, int64_t vocab, int act_tiles, hipStream_t s);
// decode.hip: kvhp_decode_attention on paged views writing its output [B][Hq*D]
// row-tiled (act_tiles = act_tiles_for(batch)); the fast kernels are
// instantiated separately for it, so row-major calls run unchanged code.
int decode_attention_act(const void* q, const kvhp_kv_view* k_view, const kvhp_kv_view* v_view,
                         const int32_t* seq_lens, void* out, int batch, int num_q_heads,
                         int num_kv_heads, int head_dim, int max_seq_len, void* workspace,
                         size_t workspace_bytes, int act_tiles, hipStream_t s);

#define KVHP_REQUIRE(cond, code, ...)          \
    do {                                       \
        if (!(cond)) return ::kvhp::fail(code, __VA_ARGS__); \
    } while (0)

#define KVHP_HIP(call, what)                                                  \
    do {                                                                      \
        hipError_t e_ = (call);                                               \
        if (e_ != hipSuccess)                                                 \
            return ::kvhp::fail(KVHP_ERR_HIP, "%s: %s", what,                 \
                                hipGetErrorString(e_));                       \
    } while (0)

inline bool aligned16(const void* p) {
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// Workgroups of `kernel` (blocks of `threads`) resident on the current
// device at once: CUs x the occupancy limit, queried once per kernel and
// block size; 0 if the runtime cannot tell.
inline int resident_workgroups(const void* kernel, int threads) {
    struct Entry {
        const void* kernel;
        int threads, n;
    };
    static std::mutex mu;
    static std::vector<Entry> cache;
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry& e : cache)
        if (e.kernel == kernel && e.threads == threads) return e.n;
    int per_cu = 0, dev = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess ||
        hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
        (void)hipGetLastError();
        per_cu = 0;
    }
    const int n = per_cu > 0 && cus > 0 ? per_cu * cus : 0;
    cache.push_back(Entry{kernel, threads, n});
    return n;
}

// -------------------------------------------------------------- device ----
// Wave64 DPP row (16-lane) butterflies.  Controls: quad_perm [1,0,3,2] = 0xB1,
// quad_perm [2,3,0,1] = 0x4E, row_half_mirror = 0x141, row_mirror = 0x140.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                           0xF, 0xF, false));
}

// Max over the 16 lanes of each DPP row; every lane of the row gets it.
__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, dpp_f32<0xB1>(x));
    x = fmaxf(x, dpp_f32<0x4E>(x));
    x = fmaxf(x, dpp_f32<0x141>(x));
    x = fmaxf(x, dpp_f32<0x140>(x));
    return x;
}

__device__ __forceinline__ float row16_sum(float x) {
    x += dpp_f32<0xB1>(x);
    x += dpp_f32<0x4E>(x);
    x += dpp_f32<0x141>(x);
    x += dpp_f32<0x140>(x);
    return x;
}

__device__ __forceinline__ float wave_max(float x) {
    x = row16_max(x);
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}

__device__ __forceinline__ float wave_sum(float x) {
    x = row16_sum(x);
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
}

// Max / sum across the four 16-lane rows of a wave with the gfx950 row
// swaps (VALU only, no LDS round trip): rows 0<->1 and 2<->3, then 01<->23.
__device__ __forceinline__ float rows4_max(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(t[0]), __uint_as_float(t[1]));
}
__device__ __forceinline__ float rows4_sum(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(t[0]) + __uint_as_float(t[1]);
}
// Full-wave sum without LDS: DPP within each 16-lane row, then row swaps.
__device__ __forceinline__ float wave_sum_fast(float x) { return rows4_sum(row16_sum(x)); }
__device__ __forceinline__ float wave_max_fast(float x) { return rows4_max(row16_max(x)); }

__device__ __forceinline__ half8 load_half8(const f16* p) {
    return *reinterpret_cast<const half8*>(p);
}

// Streaming read of data used once (KV cache rows): non-temporal hint.
__device__ __forceinline__ half8 load_half8_stream(const f16* p) {
    return __builtin_bit_cast(half8, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p)));
}

__device__ __forceinline__ void store_half8(f16* p, half8 v) {
    *reinterpret_cast<half8*>(p) = v;
}

__device__ __forceinline__ float fast_exp2(float x) {
    return __builtin_amdgcn_exp2f(x);
}

}  // namespace kvhp
