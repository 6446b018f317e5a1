// kv_view.h -- strided or paged view of one K or V cache.
//
// Mirrors engine::cuda::KVView (reference src/cuda/kv_view.h:17-31): the
// first five members are the reference's, in its order, so aggregate
// initialisation written for the reference, `KVView{ptr, sb, sh, ss, 1}`,
// still compiles and means the same strided view.  The trailing members add
// the block table that file's comment plans for (kv_view.h:9-10); left at
// their defaults the view is strided.  The struct is byte-for-byte the C
// ABI's kvhp_kv_view, so it is passed to the library without conversion.
#pragma once

#include <cstddef>
#include <cstdint>

#include "half.h"
#include "kvhp_c.h"

// Host and device qualifiers when the including file is compiled as HIP.
#ifndef KVHP_HD
#ifdef __HIPCC__
#define KVHP_HD __host__ __device__
#else
#define KVHP_HD
#endif
#endif

namespace engine {
namespace hip {

struct KVView {
    const half* data;
    int64_t stride_b;
    int64_t stride_h;
    int64_t stride_s;
    int64_t stride_d;
    // Paged mode (block_table != nullptr): pool [Hkv][num_pages][16][D],
    // position s of sequence b lives in page block_table[b*max_pages + s/16].
    const int32_t* block_table = nullptr;
    int32_t max_pages = 0;
    int32_t page_size = 0;
    int32_t num_pages = 0;
    int32_t reserved = 0;

    // The reference's address map (kv_view.h:24-30): element (b, h, s, d)
    // of a strided view, and of a paged view through its block table.  Both
    // forms run in host and device code; a paged view's block_table is read
    // where the call runs, so on the host use get_ptr_host with a host copy
    // of a device table.
    KVHP_HD const half* get_ptr(int b, int h, int s) const { return get_ptr(b, h, s, 0); }
    KVHP_HD const half* get_ptr(int b, int h, int s, int d) const {
        if (!block_table) return data + b * stride_b + h * stride_h + s * stride_s + d * stride_d;
        return paged_ptr(block_table, b, h, s, d);
    }
    // Paged (or strided) address with the block table read from
    // `table_host`, a host copy of block_table.
    const half* get_ptr_host(int b, int h, int s, int d, const int32_t* table_host) const {
        if (!block_table) return get_ptr(b, h, s, d);
        return paged_ptr(table_host, b, h, s, d);
    }

    const kvhp_kv_view* c_view() const { return reinterpret_cast<const kvhp_kv_view*>(this); }

private:
    KVHP_HD const half* paged_ptr(const int32_t* table, int b, int h, int s, int d) const {
        const int64_t page = table[(int64_t)b * max_pages + s / page_size];
        return data + h * stride_h + (page * page_size + s % page_size) * stride_s + d * stride_d;
    }
};

static_assert(sizeof(KVView) == sizeof(kvhp_kv_view), "KVView must match kvhp_kv_view");
static_assert(offsetof(KVView, stride_d) == offsetof(kvhp_kv_view, stride_d), "layout");
static_assert(offsetof(KVView, block_table) == offsetof(kvhp_kv_view, block_table), "layout");
static_assert(offsetof(KVView, num_pages) == offsetof(kvhp_kv_view, num_pages), "layout");

// Strided view of a contiguous [batch][Hkv][max_seq][D] cache (the layout
// the reference's tests build, test_attention.cpp:132-146).
inline KVView contiguous_view(const half* data, int num_kv_heads, int max_seq, int head_dim) {
    return KVView{data, (int64_t)num_kv_heads * max_seq * head_dim, (int64_t)max_seq * head_dim,
                  head_dim, 1};
}

// Paged view of a pool [Hkv][num_pages][16][D] through a device block table
// [batch][max_pages].
inline KVView paged_view(const half* pool, int num_pages, int head_dim,
                         const int32_t* block_table_dev, int max_pages) {
    KVView v{pool, 0, (int64_t)num_pages * KVHP_PAGE_SIZE * head_dim, head_dim, 1};
    v.block_table = block_table_dev;
    v.max_pages = max_pages;
    v.page_size = KVHP_PAGE_SIZE;
    v.num_pages = num_pages;
    return v;
}

}  // namespace hip
}  // namespace engine
