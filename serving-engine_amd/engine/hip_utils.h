// hip_utils.h -- device-memory and error plumbing of the C++ API.
//
// Mirrors src/common/cuda_utils.h of the reference (CUDA_CHECK :12-21,
// DeviceBuffer<T> :36-111, CudaTimer :113-146) on the HIP runtime: same
// names for the RAII buffer and its methods, same throw-on-error behaviour
// (std::runtime_error), same synchronous host copies with an overflow check.
// Host-only code: compiles with g++ (-D__HIP_PLATFORM_AMD__, ROCm include
// path) or hipcc and links libamdhip64.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdio>
#include <stdexcept>
#include <string>

#include "kvhp_c.h"

// Throws std::runtime_error on a HIP runtime error (reference CUDA_CHECK).
#define HIP_CHECK(call)                                                              \
    do {                                                                             \
        hipError_t err_ = (call);                                                    \
        if (err_ != hipSuccess) {                                                    \
            std::fprintf(stderr, "HIP error at %s:%d: %s\n", __FILE__, __LINE__,     \
                         hipGetErrorString(err_));                                   \
            throw std::runtime_error(std::string("HIP error: ") +                    \
                                     hipGetErrorString(err_));                       \
        }                                                                            \
    } while (0)

// Throws std::runtime_error when a kvhp_* call returns a non-zero status;
// the message is the library's kvhp_last_error().
#define KVHP_CHECK(call)                                                             \
    do {                                                                             \
        int st_ = (call);                                                            \
        if (st_ != KVHP_OK) {                                                        \
            throw std::runtime_error(std::string("kvhp error ") +                    \
                                     std::to_string(st_) + ": " + kvhp_last_error()); \
        }                                                                            \
    } while (0)

namespace engine {

using Stream = hipStream_t;

// RAII device allocation of `count` elements of T.  Move-only.
template <typename T>
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t count) { allocate(count); }
    ~DeviceBuffer() { reset(); }

    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;

    DeviceBuffer(DeviceBuffer&& o) noexcept : ptr_(o.ptr_), size_(o.size_) {
        o.ptr_ = nullptr;
        o.size_ = 0;
    }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) {
            reset();
            ptr_ = o.ptr_;
            size_ = o.size_;
            o.ptr_ = nullptr;
            o.size_ = 0;
        }
        return *this;
    }

    void allocate(size_t count) {
        reset();
        if (count == 0) return;
        void* p = nullptr;
        HIP_CHECK(hipMalloc(&p, count * sizeof(T)));
        ptr_ = static_cast<T*>(p);
        size_ = count;
    }

    void reset() {
        if (ptr_) {
            (void)hipFree(ptr_);
            ptr_ = nullptr;
            size_ = 0;
        }
    }

    T* data() { return ptr_; }
    const T* data() const { return ptr_; }
    size_t size() const { return size_; }
    size_t size_bytes() const { return size_ * sizeof(T); }

    // Synchronous copies, as in the reference (cuda_utils.h:90-102).
    void copy_from_host(const T* src, size_t count) {
        if (count > size_) throw std::runtime_error("DeviceBuffer::copy_from_host buffer overflow");
        if (count) HIP_CHECK(hipMemcpy(ptr_, src, count * sizeof(T), hipMemcpyHostToDevice));
    }
    void copy_to_host(T* dst, size_t count) const {
        if (count > size_) throw std::runtime_error("DeviceBuffer::copy_to_host buffer overflow");
        if (count) HIP_CHECK(hipMemcpy(dst, ptr_, count * sizeof(T), hipMemcpyDeviceToHost));
    }
    void zero() {
        if (ptr_ && size_) HIP_CHECK(hipMemset(ptr_, 0, size_ * sizeof(T)));
    }

private:
    T* ptr_ = nullptr;
    size_t size_ = 0;
};

// Event pair timing work on a stream (reference CudaTimer).
class HipTimer {
public:
    HipTimer() {
        HIP_CHECK(hipEventCreate(&start_));
        HIP_CHECK(hipEventCreate(&stop_));
    }
    ~HipTimer() {
        (void)hipEventDestroy(start_);
        (void)hipEventDestroy(stop_);
    }
    HipTimer(const HipTimer&) = delete;
    HipTimer& operator=(const HipTimer&) = delete;

    void start(Stream s = nullptr) { HIP_CHECK(hipEventRecord(start_, s)); }
    void stop(Stream s = nullptr) { HIP_CHECK(hipEventRecord(stop_, s)); }
    float elapsed_ms() {
        HIP_CHECK(hipEventSynchronize(stop_));
        float ms = 0.f;
        HIP_CHECK(hipEventElapsedTime(&ms, start_, stop_));
        return ms;
    }
    hipEvent_t get_start_event() const { return start_; }
    hipEvent_t get_stop_event() const { return stop_; }

private:
    hipEvent_t start_ = nullptr;
    hipEvent_t stop_ = nullptr;
};

// The reference's name for the timer (src/common/cuda_utils.h:116-148), so
// callers that time with it compile unchanged.
using CudaTimer = HipTimer;

}  // namespace engine
