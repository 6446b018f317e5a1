// test_kv_view_device.hip -- engine::hip::KVView::get_ptr in device code.
//
// The reference's KVView accessors are __device__ functions that kernels
// call (src/cuda/kv_view.h:24-30).  A kernel here reads elements through
// get_ptr(b, h, s, d) of a strided view (stride_d = 1 and a transposed view
// with stride_d != 1) and of a paged view whose block table is device
// memory; the host then checks every value against the element that
// get_ptr_host addresses in a host copy of the same data.  Exit status 0
// when every element matches.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "kv_view.h"

using engine::half;
using engine::hip::KVView;

#define CHECK(call)                                                                        \
    do {                                                                                   \
        hipError_t e_ = (call);                                                            \
        if (e_ != hipSuccess) {                                                            \
            std::printf("HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
            return 1;                                                                      \
        }                                                                                  \
    } while (0)

// out[((b*H + h)*S + s)*D + d] = *view.get_ptr(b, h, s, d)
__global__ void gather_kernel(KVView view, int B, int H, int S, int D, uint16_t* out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B * H * S * D) return;
    const int d = i % D;
    const int s = (i / D) % S;
    const int h = (i / (D * S)) % H;
    const int b = i / (D * S * H);
    out[i] = view.get_ptr(b, h, s, d)->bits;
}

static int run(const char* name, const KVView& dev_view, const KVView& host_view,
               const int32_t* table_host, int B, int H, int S, int D) {
    const int n = B * H * S * D;
    uint16_t* out = nullptr;
    CHECK(hipMalloc(&out, n * sizeof(uint16_t)));
    hipLaunchKernelGGL(gather_kernel, dim3((n + 255) / 256), dim3(256), 0, 0, dev_view, B, H, S, D,
                       out);
    CHECK(hipGetLastError());
    std::vector<uint16_t> got(n);
    CHECK(hipMemcpy(got.data(), out, n * sizeof(uint16_t), hipMemcpyDeviceToHost));
    CHECK(hipFree(out));
    int bad = 0;
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
            for (int s = 0; s < S; ++s)
                for (int d = 0; d < D; ++d) {
                    const uint16_t want = host_view.get_ptr_host(b, h, s, d, table_host)->bits;
                    if (got[((b * H + h) * S + s) * D + d] != want && bad++ < 5)
                        std::printf("  %s: (%d,%d,%d,%d) got %04x want %04x\n", name, b, h, s, d,
                                    got[((b * H + h) * S + s) * D + d], want);
                }
    std::printf("%s: %d elements, %d mismatches\n", name, n, bad);
    return bad ? 1 : 0;
}

int main() {
    std::mt19937 rng(2024);
    const int B = 3, H = 2, S = 40, D = 16, P = 12;
    // Random bit patterns, so that a wrong address shows.  One buffer holds
    // the strided [B][H][S][D] tensor and the paged pool [H][P][16][D] (the
    // larger).
    std::vector<half> host((size_t)H * P * 16 * D);
    for (auto& x : host) x.bits = static_cast<uint16_t>(rng());
    half* dev = nullptr;
    CHECK(hipMalloc(&dev, host.size() * sizeof(half)));
    CHECK(hipMemcpy(dev, host.data(), host.size() * sizeof(half), hipMemcpyHostToDevice));
    int fails = 0;

    // contiguous [B][H][S][D], stride_d = 1
    const KVView c_dev{dev, (int64_t)H * S * D, (int64_t)S * D, D, 1};
    const KVView c_host{host.data(), (int64_t)H * S * D, (int64_t)S * D, D, 1};
    fails += run("strided", c_dev, c_host, nullptr, B, H, S, D);

    // the same bytes read as [B][H][D][S] (stride_s = 1, stride_d = S): the
    // d * stride_d term of get_ptr(b, h, s, d)
    const KVView t_dev{dev, (int64_t)H * S * D, (int64_t)S * D, 1, S};
    const KVView t_host{host.data(), (int64_t)H * S * D, (int64_t)S * D, 1, S};
    fails += run("transposed", t_dev, t_host, nullptr, B, H, S, D);

    // paged: pool [H][P][16][D] from the same bytes, block table [B][3]
    // (a permutation of page ids, device memory for the kernel)
    std::vector<int32_t> table(B * 3);
    std::vector<int32_t> perm(P);
    for (int i = 0; i < P; ++i) perm[i] = i;
    std::shuffle(perm.begin(), perm.end(), rng);
    for (int i = 0; i < B * 3; ++i) table[i] = perm[i];
    int32_t* table_dev = nullptr;
    CHECK(hipMalloc(&table_dev, table.size() * sizeof(int32_t)));
    CHECK(hipMemcpy(table_dev, table.data(), table.size() * sizeof(int32_t), hipMemcpyHostToDevice));
    const KVView p_dev = engine::hip::paged_view(dev, P, D, table_dev, 3);
    const KVView p_host = engine::hip::paged_view(host.data(), P, D, table_dev, 3);
    fails += run("paged", p_dev, p_host, table.data(), B, H, 48, D);

    CHECK(hipFree(table_dev));
    CHECK(hipFree(dev));
    std::printf("%s\n", fails ? "FAILED" : "all ok");
    return fails ? 1 : 0;
}
