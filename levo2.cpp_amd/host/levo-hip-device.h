// Device-memory and error plumbing shared by the C++17 drop-in wrappers.
//
// The kernels behind include/levo_hip.h never allocate; these wrappers own the
// device buffers that the reference's host-vector interfaces need (the
// logits of Sampler::sample, the Euler state of solve_flow_euler) and turn the
// C ABI's status codes back into the exception types the reference throws.
#pragma once

#include "levo_hip.h"

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <functional>
#include <stdexcept>
#include <string>
#include <utility>

// The cancellation exception. Built inside the reference tree with
// -DLEVO_HIP_WITH_LEVO_H and the reference's include/ directory on the include
// path, the wrappers throw the reference's own levo::operation_cancelled
// (include/levo.h:21-24), so its catch sites (src/levo-flow-renderer.cpp:249,
// 325; src/cantor-abi.cpp:909) match unchanged. Built standalone, the library
// defines a class of its own with the same base and message.
#if defined(LEVO_HIP_WITH_LEVO_H)
#include <levo.h>

namespace levo::hip {
using operation_cancelled = ::levo::operation_cancelled;
using cancellation_callback = ::levo::cancellation_callback;
} // namespace levo::hip
#else
namespace levo::hip {
class operation_cancelled : public std::runtime_error {
public:
    operation_cancelled() : std::runtime_error("LeVo operation cancelled") {}
};

using cancellation_callback = std::function<bool()>;
} // namespace levo::hip
#endif

namespace levo::hip {

using stream_t = hipStream_t;

// Throws std::runtime_error("LeVo HIP: <what>: <HIP error>") if status is not hipSuccess.
void check_hip(hipError_t status, const char * what);

// Which exception a failing C ABI call becomes, so each wrapper throws what
// the reference function it replaces throws for the same condition.
enum class error_kind { invalid_argument, runtime_error };

// status < 0: throws `kind` carrying levo_hip_last_error() (a HIP runtime
// failure is always a std::runtime_error). Returns status otherwise.
int64_t check_status(int64_t status, error_kind kind = error_kind::invalid_argument);

// Owning device allocation of `size()` elements (hipMalloc / hipFree).
template <typename T>
class device_buffer {
public:
    device_buffer() = default;
    explicit device_buffer(std::size_t count) { allocate(count); }
    ~device_buffer() { release(); }
    device_buffer(const device_buffer &) = delete;
    device_buffer & operator=(const device_buffer &) = delete;
    device_buffer(device_buffer && other) noexcept
        : data_(std::exchange(other.data_, nullptr)), size_(std::exchange(other.size_, 0)) {}
    device_buffer & operator=(device_buffer && other) noexcept {
        if (this != &other) {
            release();
            data_ = std::exchange(other.data_, nullptr);
            size_ = std::exchange(other.size_, 0);
        }
        return *this;
    }

    T * data() noexcept { return data_; }
    const T * data() const noexcept { return data_; }
    std::size_t size() const noexcept { return size_; }

    // Grows to at least `count` elements; the old contents are not kept.
    void reserve_discard(std::size_t count) {
        if (count <= size_) return;
        release();
        allocate(count);
    }

    void upload(const T * host, std::size_t count, stream_t stream) {
        if (count > size_) throw std::logic_error("LeVo HIP: device buffer upload overflows");
        if (count == 0) return;
        check_hip(hipMemcpyAsync(data_, host, count * sizeof(T), hipMemcpyHostToDevice, stream),
                  "host-to-device copy");
    }
    void download(T * host, std::size_t count, stream_t stream) const {
        if (count > size_) throw std::logic_error("LeVo HIP: device buffer download overflows");
        if (count == 0) return;
        check_hip(hipMemcpyAsync(host, data_, count * sizeof(T), hipMemcpyDeviceToHost, stream),
                  "device-to-host copy");
    }

private:
    void allocate(std::size_t count) {
        if (count == 0) return;
        void * p = nullptr;
        check_hip(hipMalloc(&p, count * sizeof(T)), "device allocation");
        data_ = static_cast<T *>(p);
        size_ = count;
    }
    void release() noexcept {
        if (data_) (void) hipFree(data_);
        data_ = nullptr;
        size_ = 0;
    }

    T * data_ = nullptr;
    std::size_t size_ = 0;
};

// Page-locked host allocation (hipHostMalloc) for the small result copies
// that a host-side decision waits on.
template <typename T>
class pinned_buffer {
public:
    pinned_buffer() = default;
    explicit pinned_buffer(std::size_t count) { allocate(count); }
    ~pinned_buffer() { release(); }
    pinned_buffer(const pinned_buffer &) = delete;
    pinned_buffer & operator=(const pinned_buffer &) = delete;
    pinned_buffer(pinned_buffer && other) noexcept
        : data_(std::exchange(other.data_, nullptr)), size_(std::exchange(other.size_, 0)) {}
    pinned_buffer & operator=(pinned_buffer && other) noexcept {
        if (this != &other) {
            release();
            data_ = std::exchange(other.data_, nullptr);
            size_ = std::exchange(other.size_, 0);
        }
        return *this;
    }

    T * data() noexcept { return data_; }
    const T * data() const noexcept { return data_; }
    std::size_t size() const noexcept { return size_; }
    T & operator[](std::size_t i) noexcept { return data_[i]; }
    const T & operator[](std::size_t i) const noexcept { return data_[i]; }

    void reserve_discard(std::size_t count) {
        if (count <= size_) return;
        release();
        allocate(count);
    }

private:
    void allocate(std::size_t count) {
        if (count == 0) return;
        void * p = nullptr;
        check_hip(hipHostMalloc(&p, count * sizeof(T), hipHostMallocDefault), "pinned host allocation");
        data_ = static_cast<T *>(p);
        size_ = count;
    }
    void release() noexcept {
        if (data_) (void) hipHostFree(data_);
        data_ = nullptr;
        size_ = 0;
    }

    T * data_ = nullptr;
    std::size_t size_ = 0;
};

// Waits for all work enqueued on `stream`.
void synchronize(stream_t stream);

} // namespace levo::hip
