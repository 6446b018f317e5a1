// bandwidth.hip -- read-bandwidth calibration (the reference's read-bandwidth
// probe, src/cuda/read_bandwidth.cu:8-118, which calibrates its decode
// ceilings, docs/GATES.md:21).
//
// stream_read_kernel reads every 16-byte chunk of a buffer once with
// non-temporal loads: each workgroup streams its own contiguous share, eight
// 16-byte chunks in flight per lane (adjacent 4 KB blocks of the workgroup),
// and folds them into one word per lane that is stored only if it equals a
// fixed constant (so the loads cannot be dropped and nothing is written in
// practice).  Measured over 2 GiB on MI355X: a grid-stride loop (consecutive
// lanes adjacent, a lane's loads a grid apart, as the reference's probe)
// reaches ~5.9 TB/s, per-workgroup contiguous shares ~6.9-7.0 TB/s, and plain
// (temporal) loads ~1 TB/s less than non-temporal ones; the contiguous form
// is the device's streaming-read ceiling.
//
// page_read_kernel reads a list of pages (2 or 4 KB: the page of one KV head
// at D = 64 or 128; up to 32 KB to measure coarser layouts) in list order,
// one wave per workgroup, 16 KB of pages in flight per wave: the ceiling of
// a paged decode that reads the same pages in a random order.
#include "kvhp_internal.h"

#include <algorithm>

namespace kvhp {
namespace {

constexpr int kReadThreads = 256;
constexpr uint32_t kSinkMagic = 0x9E3779B9u;

constexpr int kReadDepth = 8;   // 16-byte chunks in flight per lane

__global__ void __launch_bounds__(kReadThreads)
stream_read_kernel(const u32x4* p, size_t n16, uint32_t* sink) {
    const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const size_t beg = (size_t)blockIdx.x * per;
    const size_t end = beg + per < n16 ? beg + per : n16;
    size_t i = beg + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (kReadDepth - 1) * kReadThreads < end; i += kReadDepth * kReadThreads) {
        u32x4 v[kReadDepth];
#pragma unroll
        for (int j = 0; j < kReadDepth; ++j) v[j] = __builtin_nontemporal_load(p + i + j * kReadThreads);
#pragma unroll
        for (int j = 0; j < kReadDepth; ++j) acc ^= (v[j][0] + v[j][1]) ^ (v[j][2] + v[j][3] + j);
    }
    for (; i < end; i += kReadThreads) {
        const u32x4 a = __builtin_nontemporal_load(p + i);
        acc ^= a[0] + a[1] + a[2] + a[3];
    }
    if (acc == kSinkMagic) *sink = acc;
}

// LPP: 1 KB wave loads per page (2 to 32: pages of 2 to 32 KB), PIF pages in
// flight per wave (16 KB in flight, at least one page).  Wave w reads list
// entries [w*per, (w+1)*per); ids outside the pool are clamped into it.
template <int LPP>
__global__ void __launch_bounds__(kWave)
page_read_kernel(const u32x4* pool, int64_t pool_pages, const int32_t* ids, int64_t n_ids,
                 int64_t per, uint32_t* sink) {
    constexpr int kPagesInFlight = LPP >= 16 ? 1 : 16 / LPP;
    const int lane = threadIdx.x;
    const int64_t beg = (int64_t)blockIdx.x * per;
    const int64_t end = beg + per < n_ids ? beg + per : n_ids;
    uint32_t acc = 0;
    for (int64_t i = beg; i < end; i += kPagesInFlight) {
        u32x4 v[kPagesInFlight][LPP];
#pragma unroll
        for (int j = 0; j < kPagesInFlight; ++j) {
            const int64_t e = i + j < end ? i + j : end - 1;
            int64_t id = ids[e];
            id = id < 0 ? 0 : (id >= pool_pages ? pool_pages - 1 : id);
            const u32x4* pg = pool + id * (LPP * kWave);
#pragma unroll
            for (int r = 0; r < LPP; ++r) v[j][r] = __builtin_nontemporal_load(pg + r * kWave + lane);
        }
#pragma unroll
        for (int j = 0; j < kPagesInFlight; ++j)
#pragma unroll
            for (int r = 0; r < LPP; ++r) acc ^= (v[j][r][0] + v[j][r][1]) ^ (v[j][r][2] + v[j][r][3] + j);
    }
    if (acc == kSinkMagic) *sink = acc;
}

}  // namespace
}  // namespace kvhp

using namespace kvhp;

extern "C" int kvhp_stream_read(const void* buf, size_t bytes, void* sink, void* stream) {
    clear_error();
    if (bytes < 16) return KVHP_OK;
    KVHP_REQUIRE(buf && sink, KVHP_ERR_INVALID, "stream_read: null pointer");
    KVHP_REQUIRE(aligned16(buf), KVHP_ERR_INVALID, "stream_read: buffer not 16-byte aligned");
    // eight resident 256-lane workgroups per CU fill the device's wave slots
    int dev = 0, cus = 0;
    KVHP_HIP(hipGetDevice(&dev), "hipGetDevice");
    KVHP_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev),
             "hipDeviceGetAttribute");
    const size_t n16 = bytes / 16;
    const size_t want = (size_t)(cus > 0 ? cus : 256) * 8;
    const size_t blocks = std::min(want, (n16 + kReadThreads - 1) / kReadThreads);
    hipLaunchKernelGGL(stream_read_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kReadThreads),
                       0, static_cast<hipStream_t>(stream), static_cast<const u32x4*>(buf), n16,
                       static_cast<uint32_t*>(sink));
    return check_launch("stream_read");
}

extern "C" int kvhp_page_read(const void* pool, int64_t pool_bytes, const int32_t* page_ids,
                              int64_t n_ids, int page_bytes, void* sink, void* stream) {
    clear_error();
    if (n_ids <= 0) return KVHP_OK;
    KVHP_REQUIRE(pool && page_ids && sink, KVHP_ERR_INVALID, "page_read: null pointer");
    KVHP_REQUIRE(aligned16(pool), KVHP_ERR_INVALID, "page_read: pool not 16-byte aligned");
    KVHP_REQUIRE(page_bytes == 2048 || page_bytes == 4096 || page_bytes == 8192 ||
                     page_bytes == 16384 || page_bytes == 32768,
                 KVHP_ERR_UNSUPPORTED, "page_read: page_bytes %d is not a power of two in 2..32 KB",
                 page_bytes);
    const int64_t pool_pages = pool_bytes / page_bytes;
    KVHP_REQUIRE(pool_pages > 0, KVHP_ERR_INVALID, "page_read: pool smaller than a page");
    int dev = 0, cus = 0;
    KVHP_HIP(hipGetDevice(&dev), "hipGetDevice");
    KVHP_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev),
             "hipDeviceGetAttribute");
    // eight waves per CU, each a contiguous share of the list (16 KB of
    // pages per wave at a time)
    const int pif = page_bytes >= 16384 ? 1 : 16384 / page_bytes;
    const int64_t want = (int64_t)(cus > 0 ? cus : 256) * 8;
    const int64_t waves = std::min<int64_t>(want, (n_ids + pif - 1) / pif);
    const int64_t per = (n_ids + waves - 1) / waves;
    const int64_t grid = (n_ids + per - 1) / per;
    auto* p = static_cast<const u32x4*>(pool);
    auto* sk = static_cast<uint32_t*>(sink);
    auto s = static_cast<hipStream_t>(stream);
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(grid)), dim3(kWave), 0, s, p,
                           pool_pages, page_ids, n_ids, per, sk);
    };
    switch (page_bytes) {
        case 2048: go(page_read_kernel<2>); break;
        case 4096: go(page_read_kernel<4>); break;
        case 8192: go(page_read_kernel<8>); break;
        case 16384: go(page_read_kernel<16>); break;
        default: go(page_read_kernel<32>); break;
    }
    return check_launch("page_read");
}
