// kv_append.hip -- KV-cache writes and the paged gather (bit-exact copies).
//
// Layout: every kernel moves 16-byte vectors (8 fp16).  Appends of 16 or
// more tokens go by runs (one wave per 16 tokens of one KV head: a page's
// worth of rows, all loads before the stores); shorter ones and the generic
// gather by chunks (one work item is one 16-byte chunk of a K row plus the
// same chunk of the V row, fully coalesced, 16-byte aligned); the paged
// gather by pages.
// These kernels are HBM-bound byte copies: algorithmic traffic is exactly
// 2 (read+write) x 2 (K,V) x T*Hkv*D*2 bytes (+4 B per block-table lookup).
// A scalar (2-byte) variant handles head dims that are not multiples of 8.
#include "kvhp_internal.h"

#include <algorithm>

namespace kvhp {

namespace {

constexpr int kCopyThreads = 256;

// Contiguous append, same index map as the reference append_kv_kernel
// (src/runtime/kv_cache.cu:20-35): src (t*Hkv + h)*D + d ->
// dst (h*max_seq + start_pos + t)*D + d, positions >= max_seq skipped (:26).
template <int VEC>
__global__ void __launch_bounds__(kCopyThreads)
append_contig_kernel(const f16* __restrict__ src_k, const f16* __restrict__ src_v,
                     f16* __restrict__ dst_k, f16* __restrict__ dst_v,
                     int64_t n_chunks, int chunks_per_row, int num_kv_heads,
                     int start_pos, int max_seq, int head_dim) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n_chunks;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / chunks_per_row;          // t*Hkv + h
        const int c = static_cast<int>(i - row * chunks_per_row);
        const int t = static_cast<int>(row / num_kv_heads);
        const int h = static_cast<int>(row - (int64_t)t * num_kv_heads);
        const int pos = start_pos + t;
        if (pos < 0 || pos >= max_seq) continue;
        const int64_t so = row * head_dim + (int64_t)c * VEC;
        const int64_t dofs = ((int64_t)h * max_seq + pos) * head_dim + (int64_t)c * VEC;
        if constexpr (VEC == 8) {
            store_half8(dst_k + dofs, load_half8(src_k + so));
            store_half8(dst_v + dofs, load_half8(src_v + so));
        } else {
            dst_k[dofs] = src_k[so];
            dst_v[dofs] = src_v[so];
        }
    }
}

// Paged append: token (b,t) at position start_pos[b]+t lands in
// pool[h][bt[b][pos/16]][pos%16][:].
template <int VEC>
__global__ void __launch_bounds__(kCopyThreads)
append_paged_kernel(const f16* __restrict__ src_k, const f16* __restrict__ src_v,
                    f16* __restrict__ pool_k, f16* __restrict__ pool_v,
                    const int32_t* __restrict__ block_tables, int max_pages,
                    const int32_t* __restrict__ start_pos, int64_t n_chunks,
                    int chunks_per_row, int num_tokens, int num_kv_heads,
                    int head_dim, int num_pages) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n_chunks;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / chunks_per_row;          // (b*T + t)*Hkv + h
        const int c = static_cast<int>(i - row * chunks_per_row);
        const int64_t bt_row = row / num_kv_heads;       // b*T + t
        const int h = static_cast<int>(row - bt_row * num_kv_heads);
        const int b = static_cast<int>(bt_row / num_tokens);
        const int t = static_cast<int>(bt_row - (int64_t)b * num_tokens);
        const int pos = start_pos[b] + t;
        if (pos < 0) continue;
        const int pi = pos / kPage;
        if (pi >= max_pages) continue;
        const int pid = block_tables[(int64_t)b * max_pages + pi];
        if (pid < 0 || pid >= num_pages) continue;
        const int64_t so = row * head_dim + (int64_t)c * VEC;
        const int64_t dofs =
            (((int64_t)h * num_pages + pid) * kPage + (pos % kPage)) * head_dim +
            (int64_t)c * VEC;
        if constexpr (VEC == 8) {
            store_half8(pool_k + dofs, load_half8(src_k + so));
            store_half8(pool_v + dofs, load_half8(src_v + so));
        } else {
            pool_k[dofs] = src_k[so];
            pool_v[dofs] = src_v[so];
        }
    }
}

// Append by runs (prompt-sized T): one wave moves a run of 16 consecutive
// tokens of one KV head, K and V.  The run's source rows are D-element
// pieces of the token-major [B][T][Hkv][D] input (row pitch Hkv*D); they land
// as 16 consecutive rows of the destination -- one 32*D-byte page when the
// run starts on a page boundary (prefill from position 0), two pages
// otherwise, or 16 consecutive rows of the head-major contiguous cache.
// CPL = D/32 16-byte chunks per lane and tensor, every load of the run in
// flight before its stores; unit indices and row/column splits are 32-bit
// shifts and masks (no 64-bit division per chunk).  Units run KV head
// fastest, so a workgroup's four waves read the same tokens' rows.  Each
// destination row is written by exactly the lanes that loaded it, with the
// same drop rules as the chunk kernels: positions >= max_seq (contiguous),
// or negative, past max_pages, or whose page id lies outside the pool
// (paged).
template <int CPL, bool PAGED>
__global__ void __launch_bounds__(kCopyThreads)
append_runs_kernel(const f16* __restrict__ src_k, const f16* __restrict__ src_v,
                   f16* __restrict__ dst_k, f16* __restrict__ dst_v,
                   const int32_t* __restrict__ block_tables, int max_pages,
                   const int32_t* __restrict__ start_pos_dev, int start_pos, int num_units,
                   int runs_per_seq, int num_tokens, int num_kv_heads, int max_seq,
                   int num_pages) {
    constexpr int D = 32 * CPL;
    constexpr int CPR = D / 8;                        // 16-byte chunks per row
    constexpr int RSH = CPR == 4 ? 2 : CPR == 8 ? 3 : CPR == 16 ? 4 : 5;
    static_assert((1 << RSH) == CPR, "chunks per row must be 4..32");
    const int lane = threadIdx.x & (kWave - 1);
    const int nwaves = static_cast<int>(((int64_t)gridDim.x * blockDim.x) >> 6);
    for (int u = static_cast<int>(((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6);
         u < num_units; u += nwaves) {
        const int h = u % num_kv_heads;
        const int br = u / num_kv_heads;              // b * runs_per_seq + r
        const int b = br / runs_per_seq;
        const int t0 = kPage * (br - b * runs_per_seq);
        const int p0 = (PAGED ? start_pos_dev[b] : start_pos) + t0;
        int64_t so[CPL], dofs[CPL];
        bool ok[CPL];
        half8 kx[CPL], vx[CPL];
        // The source loads depend on the token index only; the destination's
        // page id is loaded alongside them and checked at the store, so the
        // K/V loads never wait for the block table.
        int pid[CPL];
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + kWave * i;
            const int row = c >> RSH;
            const int col = c & (CPR - 1);
            const int t = t0 + row;
            const int pos = p0 + row;
            const bool src_ok = t < num_tokens;
            bool v = src_ok && pos >= 0;
            pid[i] = -1;
            if constexpr (PAGED) {
                const int pi = pos >> 4;
                if (v && pi < max_pages) pid[i] = block_tables[(int64_t)b * max_pages + pi];
                dofs[i] = ((int64_t)h * num_pages * kPage + (pos & (kPage - 1))) * D + 8 * col;
            } else {
                v = v && pos < max_seq;
                dofs[i] = ((int64_t)h * max_seq + pos) * D + 8 * col;
            }
            ok[i] = v;
            so[i] = (((int64_t)b * num_tokens + t) * num_kv_heads + h) * D + 8 * col;
            kx[i] = src_ok ? load_half8(src_k + so[i]) : half8{};
            vx[i] = src_ok ? load_half8(src_v + so[i]) : half8{};
        }
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            bool v = ok[i];
            int64_t o = dofs[i];
            if constexpr (PAGED) {
                v = v && pid[i] >= 0 && pid[i] < num_pages;
                o += (int64_t)pid[i] * kPage * D;
            }
            if (v) {
                store_half8(dst_k + o, kx[i]);
                store_half8(dst_v + o, vx[i]);
            }
        }
    }
}

// Launch of append_runs_kernel for D in {32, 64, 128, 256} (16-byte aligned
// tensors); false when the shape needs the chunk kernels.
template <bool PAGED>
bool launch_append_runs(const void* src_k, const void* src_v, void* dst_k, void* dst_v,
                        const int32_t* bt, int max_pages, const int32_t* start_dev,
                        int start_host, int batch, int num_tokens, int num_kv_heads,
                        int head_dim, int max_seq, int num_pages, hipStream_t s) {
    const int runs = (num_tokens + kPage - 1) / kPage;
    const int64_t units = (int64_t)batch * runs * num_kv_heads;
    if (units > (int64_t)1 << 30) return false;
    const int64_t blocks = std::min<int64_t>((units + 3) / 4, 256 * 64);
    const dim3 grid(static_cast<unsigned>(std::max<int64_t>(blocks, 1)));
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(kCopyThreads), 0, s, (const f16*)src_k,
                           (const f16*)src_v, (f16*)dst_k, (f16*)dst_v, bt, max_pages,
                           start_dev, start_host, static_cast<int>(units), runs, num_tokens,
                           num_kv_heads, max_seq, num_pages);
    };
    switch (head_dim) {
        case 32: go(append_runs_kernel<1, PAGED>); return true;
        case 64: go(append_runs_kernel<2, PAGED>); return true;
        case 128: go(append_runs_kernel<4, PAGED>); return true;
        case 256: go(append_runs_kernel<8, PAGED>); return true;
        default: return false;
    }
}

// Paged gather: out[b][h][s][:] = pool[h][bt[b][s/16]][s%16][:] for
// s < seq_lens[b], zero elsewhere (and for ids outside the pool).
template <int VEC>
__global__ void __launch_bounds__(kCopyThreads)
gather_paged_kernel(const f16* __restrict__ pool_k, const f16* __restrict__ pool_v,
                    const int32_t* __restrict__ block_tables, int max_pages,
                    const int32_t* __restrict__ seq_lens, int64_t n_chunks,
                    int chunks_per_row, int max_len, int num_kv_heads,
                    int head_dim, int num_pages, f16* __restrict__ out_k,
                    f16* __restrict__ out_v) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n_chunks;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / chunks_per_row;          // (b*Hkv + h)*max_len + s
        const int c = static_cast<int>(i - row * chunks_per_row);
        const int64_t bh = row / max_len;
        const int s = static_cast<int>(row - bh * max_len);
        const int b = static_cast<int>(bh / num_kv_heads);
        const int h = static_cast<int>(bh - (int64_t)b * num_kv_heads);
        const int64_t o = row * head_dim + (int64_t)c * VEC;
        int pid = -1;
        if (s < seq_lens[b] && s / kPage < max_pages)
            pid = block_tables[(int64_t)b * max_pages + s / kPage];
        if (pid < 0 || pid >= num_pages) {
            if constexpr (VEC == 8) {
                const half8 z = {};
                store_half8(out_k + o, z);
                store_half8(out_v + o, z);
            } else {
                out_k[o] = f16(0);
                out_v[o] = f16(0);
            }
            continue;
        }
        const int64_t src =
            (((int64_t)h * num_pages + pid) * kPage + (s % kPage)) * head_dim +
            (int64_t)c * VEC;
        if constexpr (VEC == 8) {
            store_half8(out_k + o, load_half8(pool_k + src));
            store_half8(out_v + o, load_half8(pool_v + src));
        } else {
            out_k[o] = pool_k[src];
            out_v[o] = pool_v[src];
        }
    }
}

// Paged gather by pages: one wave per (sequence, KV head, page) moves the
// page's 16 rows of K and of V (32*D contiguous bytes each, in the pool and
// in the output alike), CPL = D/32 16-byte chunks per lane and tensor, all
// loads of both tensors in flight before the stores; one block-table
// lookup per page.  Rows at or past seq_lens[b], and pages outside the
// pool, are written as zeros; rows past max_len are not written.
template <int CPL>
__global__ void __launch_bounds__(kCopyThreads)
gather_pages_kernel(const f16* __restrict__ pool_k, const f16* __restrict__ pool_v,
                    const int32_t* __restrict__ block_tables, int max_pages,
                    const int32_t* __restrict__ seq_lens, int64_t n_units, int pages_per_seq,
                    int max_len, int num_kv_heads, int num_pages, f16* __restrict__ out_k,
                    f16* __restrict__ out_v) {
    constexpr int D = 32 * CPL;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
    for (int64_t u = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6; u < n_units;
         u += nwaves) {
        const int p = static_cast<int>(u % pages_per_seq);
        const int64_t bh = u / pages_per_seq;          // b * Hkv + h
        const int h = static_cast<int>(bh % num_kv_heads);
        const int b = static_cast<int>(bh / num_kv_heads);
        const int L = seq_lens[b];
        int pid = -1;
        if (kPage * p < L && p < max_pages) pid = block_tables[(int64_t)b * max_pages + p];
        const bool ok = pid >= 0 && pid < num_pages;
        const int64_t src = ok ? ((int64_t)h * num_pages + pid) * kPage * D : 0;
        const int64_t dst = (bh * max_len + (int64_t)kPage * p) * D;
        half8 kx[CPL], vx[CPL];
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + kWave * i;            // chunk of the page: row 8c / D
            const bool valid = ok && kPage * p + (8 * c) / D < L;
            kx[i] = valid ? load_half8_stream(pool_k + src + 8 * c) : half8{};
            vx[i] = valid ? load_half8_stream(pool_v + src + 8 * c) : half8{};
        }
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + kWave * i;
            if (kPage * p + (8 * c) / D < max_len) {
                store_half8(out_k + dst + 8 * c, kx[i]);
                store_half8(out_v + dst + 8 * c, vx[i]);
            }
        }
    }
}

// Grid for a grid-stride copy: enough waves to cover HBM latency on 256 CUs,
// capped so very large copies loop instead of launching millions of groups.
inline unsigned copy_grid(int64_t n_items) {
    int64_t blocks = (n_items + kCopyThreads - 1) / kCopyThreads;
    const int64_t cap = 256 * 32;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    return static_cast<unsigned>(blocks);
}

}  // namespace

}  // namespace kvhp

using namespace kvhp;

extern "C" int kvhp_append_kv(const void* src_k, const void* src_v,
                              void* dst_k_head_base, void* dst_v_head_base,
                              int num_tokens, int start_pos, int num_kv_heads,
                              int max_seq, int head_dim, void* stream) {
    clear_error();
    if (num_tokens <= 0) return KVHP_OK;  // kv_cache.cu:50
    KVHP_REQUIRE(src_k && src_v && dst_k_head_base && dst_v_head_base,
                 KVHP_ERR_INVALID, "append_kv: null pointer");
    KVHP_REQUIRE(num_kv_heads > 0 && head_dim > 0 && max_seq > 0 && start_pos >= 0,
                 KVHP_ERR_INVALID,
                 "append_kv: bad shape (Hkv=%d D=%d max_seq=%d start=%d)",
                 num_kv_heads, head_dim, max_seq, start_pos);
    const bool vec = head_dim % 8 == 0 && aligned16(src_k) && aligned16(src_v) &&
                     aligned16(dst_k_head_base) && aligned16(dst_v_head_base);
    const int vw = vec ? 8 : 1;
    const int cpr = head_dim / vw;
    const int64_t n = (int64_t)num_tokens * num_kv_heads * cpr;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // prompt-sized appends by 16-token runs; a few tokens by 16-byte chunks
    // (a run of one token would leave most of a wave's lanes idle)
    if (vec && num_tokens >= kPage &&
        launch_append_runs<false>(src_k, src_v, dst_k_head_base, dst_v_head_base, nullptr, 0,
                                  nullptr, start_pos, 1, num_tokens, num_kv_heads, head_dim,
                                  max_seq, 0, s))
        return check_launch("append_kv");
    if (vec)
        hipLaunchKernelGGL(append_contig_kernel<8>, dim3(copy_grid(n)), dim3(kCopyThreads),
                           0, s, (const f16*)src_k, (const f16*)src_v,
                           (f16*)dst_k_head_base, (f16*)dst_v_head_base, n, cpr,
                           num_kv_heads, start_pos, max_seq, head_dim);
    else
        hipLaunchKernelGGL(append_contig_kernel<1>, dim3(copy_grid(n)), dim3(kCopyThreads),
                           0, s, (const f16*)src_k, (const f16*)src_v,
                           (f16*)dst_k_head_base, (f16*)dst_v_head_base, n, cpr,
                           num_kv_heads, start_pos, max_seq, head_dim);
    return check_launch("append_kv");
}

extern "C" int kvhp_paged_append_kv(const void* src_k, const void* src_v,
                                    void* pool_k, void* pool_v,
                                    const int32_t* block_tables, int max_pages,
                                    const int32_t* start_pos, int batch,
                                    int num_tokens, int num_kv_heads,
                                    int head_dim, int num_pages, void* stream) {
    clear_error();
    if (num_tokens <= 0 || batch <= 0) return KVHP_OK;
    KVHP_REQUIRE(src_k && src_v && pool_k && pool_v && block_tables && start_pos,
                 KVHP_ERR_INVALID, "paged_append_kv: null pointer");
    KVHP_REQUIRE(num_kv_heads > 0 && head_dim > 0 && max_pages > 0 && num_pages > 0,
                 KVHP_ERR_INVALID,
                 "paged_append_kv: bad shape (Hkv=%d D=%d max_pages=%d pages=%d)",
                 num_kv_heads, head_dim, max_pages, num_pages);
    const bool vec = head_dim % 8 == 0 && aligned16(src_k) && aligned16(src_v) &&
                     aligned16(pool_k) && aligned16(pool_v);
    const int vw = vec ? 8 : 1;
    const int cpr = head_dim / vw;
    const int64_t n = (int64_t)batch * num_tokens * num_kv_heads * cpr;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (vec && num_tokens >= kPage &&
        launch_append_runs<true>(src_k, src_v, pool_k, pool_v, block_tables, max_pages,
                                 start_pos, 0, batch, num_tokens, num_kv_heads, head_dim, 0,
                                 num_pages, s))
        return check_launch("paged_append_kv");
    if (vec)
        hipLaunchKernelGGL(append_paged_kernel<8>, dim3(copy_grid(n)), dim3(kCopyThreads),
                           0, s, (const f16*)src_k, (const f16*)src_v, (f16*)pool_k,
                           (f16*)pool_v, block_tables, max_pages, start_pos, n, cpr,
                           num_tokens, num_kv_heads, head_dim, num_pages);
    else
        hipLaunchKernelGGL(append_paged_kernel<1>, dim3(copy_grid(n)), dim3(kCopyThreads),
                           0, s, (const f16*)src_k, (const f16*)src_v, (f16*)pool_k,
                           (f16*)pool_v, block_tables, max_pages, start_pos, n, cpr,
                           num_tokens, num_kv_heads, head_dim, num_pages);
    return check_launch("paged_append_kv");
}

extern "C" int kvhp_paged_gather_kv(const void* pool_k, const void* pool_v,
                                    const int32_t* block_tables, int max_pages,
                                    const int32_t* seq_lens, int batch,
                                    int num_kv_heads, int head_dim,
                                    int num_pages, int max_len, void* out_k,
                                    void* out_v, void* stream) {
    clear_error();
    if (batch <= 0 || max_len <= 0) return KVHP_OK;
    KVHP_REQUIRE(pool_k && pool_v && block_tables && seq_lens && out_k && out_v,
                 KVHP_ERR_INVALID, "paged_gather_kv: null pointer");
    KVHP_REQUIRE(num_kv_heads > 0 && head_dim > 0 && max_pages > 0 && num_pages > 0,
                 KVHP_ERR_INVALID,
                 "paged_gather_kv: bad shape (Hkv=%d D=%d max_pages=%d pages=%d)",
                 num_kv_heads, head_dim, max_pages, num_pages);
    const bool vec = head_dim % 8 == 0 && aligned16(pool_k) && aligned16(pool_v) &&
                     aligned16(out_k) && aligned16(out_v);
    const int vw = vec ? 8 : 1;
    const int cpr = head_dim / vw;
    const int64_t n = (int64_t)batch * num_kv_heads * max_len * cpr;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (vec && (head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256)) {
        const int pps = (max_len + kPage - 1) / kPage;
        const int64_t units = (int64_t)batch * num_kv_heads * pps;
        const int64_t blocks = std::min<int64_t>((units + 3) / 4, 256 * 64);
        const dim3 grid(static_cast<unsigned>(std::max<int64_t>(blocks, 1)));
        auto args = [&](auto kern) {
            hipLaunchKernelGGL(kern, grid, dim3(kCopyThreads), 0, s, (const f16*)pool_k,
                               (const f16*)pool_v, block_tables, max_pages, seq_lens, units, pps,
                               max_len, num_kv_heads, num_pages, (f16*)out_k, (f16*)out_v);
        };
        if (head_dim == 32) args(gather_pages_kernel<1>);
        else if (head_dim == 64) args(gather_pages_kernel<2>);
        else if (head_dim == 128) args(gather_pages_kernel<4>);
        else args(gather_pages_kernel<8>);
        return check_launch("paged_gather_kv");
    }
    if (vec)
        hipLaunchKernelGGL(gather_paged_kernel<8>, dim3(copy_grid(n)), dim3(kCopyThreads),
                           0, s, (const f16*)pool_k, (const f16*)pool_v, block_tables,
                           max_pages, seq_lens, n, cpr, max_len, num_kv_heads,
                           head_dim, num_pages, (f16*)out_k, (f16*)out_v);
    else
        hipLaunchKernelGGL(gather_paged_kernel<1>, dim3(copy_grid(n)), dim3(kCopyThreads),
                           0, s, (const f16*)pool_k, (const f16*)pool_v, block_tables,
                           max_pages, seq_lens, n, cpr, max_len, num_kv_heads,
                           head_dim, num_pages, (f16*)out_k, (f16*)out_v);
    return check_launch("paged_gather_kv");
}
