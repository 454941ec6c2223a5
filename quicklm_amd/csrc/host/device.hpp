// Device memory and stream ownership over the kernel library's C ABI
// (include/qlm_hip.h). The engine includes no HIP header: every device
// interaction goes through qlm_* calls.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>

#include "qlm_hip.h"

namespace qlm {

inline void check(int rc, const char* what) {
    if (rc != QLM_OK)
        throw std::runtime_error(std::string(what) + ": " + qlm_error_string(rc) + " (" +
                                 std::to_string(rc) + ")");
}

// Owned device allocation (move-only).
class DeviceBuffer {
   public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes) { alloc(bytes); }
    ~DeviceBuffer() { release(); }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept : p_(o.p_), n_(o.n_) { o.p_ = nullptr, o.n_ = 0; }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) {
            release();
            p_ = o.p_, n_ = o.n_;
            o.p_ = nullptr, o.n_ = 0;
        }
        return *this;
    }
    void alloc(size_t bytes) {
        release();
        check(qlm_malloc(&p_, bytes), "qlm_malloc");
        n_ = bytes;
    }
    void release() {
        if (p_) qlm_free(p_);
        p_ = nullptr;
        n_ = 0;
    }
    template <typename T = void>
    T* get() const { return static_cast<T*>(p_); }
    size_t bytes() const { return n_; }
    explicit operator bool() const { return p_ != nullptr; }

   private:
    void* p_ = nullptr;
    size_t n_ = 0;
};

}  // namespace qlm
