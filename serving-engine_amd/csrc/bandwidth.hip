// bandwidth.hip -- streaming-read calibration (the reference's read-bandwidth
// probe, src/cuda/read_bandwidth.cu:8-118, which calibrates its decode
// ceilings, docs/GATES.md:21).
//
// stream_read_kernel reads every 16-byte chunk of a buffer once with
// non-temporal loads, four chunks in flight per lane, grid-stride, and folds
// them into one word per lane that is stored only if it equals a fixed
// constant (so the loads cannot be dropped and nothing is written in
// practice).  Its rate over a buffer far larger than the 256 MB MALL, with
// the caches flushed before it, is the read ceiling an HBM-bound kernel can
// reach on the device; the bench reports decode bytes against it beside the
// 8 TB/s specification.
#include "kvhp_internal.h"

#include <algorithm>

namespace kvhp {
namespace {

constexpr int kReadThreads = 256;
constexpr uint32_t kSinkMagic = 0x9E3779B9u;

__global__ void __launch_bounds__(kReadThreads)
stream_read_kernel(const u32x4* p, size_t n16, uint32_t* sink) {
    const size_t stride = (size_t)gridDim.x * kReadThreads;
    size_t i = (size_t)blockIdx.x * kReadThreads + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const u32x4 a = __builtin_nontemporal_load(p + i);
        const u32x4 b = __builtin_nontemporal_load(p + i + stride);
        const u32x4 c = __builtin_nontemporal_load(p + i + 2 * stride);
        const u32x4 d = __builtin_nontemporal_load(p + i + 3 * stride);
        acc ^= (a[0] ^ b[1] ^ c[2] ^ d[3]) + (a[1] ^ b[2] ^ c[3] ^ d[0]) +
               (a[2] ^ b[3] ^ c[0] ^ d[1]) + (a[3] ^ b[0] ^ c[1] ^ d[2]);
    }
    for (; i < n16; i += stride) {
        const u32x4 a = __builtin_nontemporal_load(p + i);
        acc ^= a[0] + a[1] + a[2] + a[3];
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
