// mtensor.hpp — device tensor handle of the host layer.
//
// Plays the role of the reference's MTensor (core/metal/metal_tensor.hpp:
// a retained buffer + shape, non-owning view(n)) over HIP device memory from
// msplat_hip_alloc.  Copies share the allocation (reference counted, freed
// with the last owner); view(n) aliases the first n rows and keeps the
// allocation alive.
#pragma once

#include <cstdint>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/msplat_hip.h"

namespace msplat {

enum class DType { Float32, Int32 };

inline size_t dtype_size(DType) { return 4; }

// Throws with the library's last error message when a C-ABI call fails.
inline void check(int rc, const char* what) {
    if (rc != MSPLAT_OK) {
        const char* m = msplat_hip_last_error();
        throw std::runtime_error(std::string(what) + ": " + (m ? m : "error"));
    }
}

class MTensor {
public:
    MTensor() = default;

    bool defined() const { return static_cast<bool>(mem_); }
    void reset() { mem_.reset(); ptr_ = nullptr; shape_.clear(); }

    const std::vector<int64_t>& shape() const { return shape_; }
    int64_t size(int d) const { return shape_.at(d < 0 ? shape_.size() + d : d); }
    int64_t dim() const { return (int64_t)shape_.size(); }
    int64_t numel() const {
        int64_t n = 1;
        for (int64_t s : shape_) n *= s;
        return shape_.empty() ? 0 : n;
    }
    int64_t stride0() const { return shape_.empty() || shape_[0] == 0 ? 0 : numel() / shape_[0]; }
    size_t nbytes() const { return (size_t)numel() * dtype_size(dtype_); }
    DType dtype() const { return dtype_; }

    void* data_ptr() const { return ptr_; }
    template <typename T> T* data() const { return static_cast<T*>(ptr_); }

    // First n rows, sharing the allocation.
    MTensor view(int64_t n) const {
        MTensor v = *this;
        if (!v.shape_.empty()) v.shape_[0] = n;
        return v;
    }

    // Small tensors (at most kMappedBytes) live in coherent host memory
    // mapped into the device's address space, like the reference's
    // shared-storage buffers: data() is then valid on the host too, and the
    // host reads and writes it directly.
    static constexpr size_t kMappedBytes = 256;
    bool mapped() const { return mapped_; }

    // Copies and fills keep the stream order for every tensor (a mapped one
    // waits for the stream first).
    void zero() {
        if (!numel()) return;
        if (mapped_) {
            check(msplat_hip_sync(), "sync");
            std::memset(ptr_, 0, nbytes());
        } else {
            check(msplat_hip_memset(ptr_, 0, nbytes()), "memset");
        }
    }
    void copy_from_host(const void* src, size_t bytes) {
        if (!bytes) return;
        if (mapped_) {
            check(msplat_hip_sync(), "sync");
            std::memcpy(ptr_, src, bytes);
        } else {
            check(msplat_hip_memcpy_h2d(ptr_, src, bytes), "memcpy h2d");
        }
    }
    void copy_to_host(void* dst, size_t bytes) const {
        if (!bytes) return;
        if (mapped_) {
            check(msplat_hip_sync(), "sync");
            std::memcpy(dst, ptr_, bytes);
        } else {
            check(msplat_hip_memcpy_d2h(dst, ptr_, bytes), "memcpy d2h");
        }
    }
    void copy_from_device(const void* src, size_t bytes) {
        if (bytes) check(msplat_hip_memcpy_d2d(ptr_, src, bytes), "memcpy d2d");
    }

    static MTensor empty(std::vector<int64_t> shape, DType dt) {
        MTensor t;
        t.shape_ = std::move(shape);
        t.dtype_ = dt;
        size_t bytes = (size_t)t.numel() * dtype_size(dt);
        void* p = nullptr;
        if (bytes <= kMappedBytes) {
            check(msplat_hip_alloc_mapped(&p, bytes ? bytes : 16), "alloc mapped");
            t.mem_ = std::shared_ptr<void>(p, [](void* q) { msplat_hip_free_mapped(q); });
            t.mapped_ = true;
        } else {
            check(msplat_hip_alloc(&p, bytes), "alloc");
            t.mem_ = std::shared_ptr<void>(p, [](void* q) { msplat_hip_free(q); });
        }
        t.ptr_ = p;
        return t;
    }
    static MTensor zeros(std::vector<int64_t> shape, DType dt) {
        MTensor t = empty(std::move(shape), dt);
        t.zero();
        return t;
    }

private:
    std::shared_ptr<void> mem_;
    void* ptr_ = nullptr;
    bool mapped_ = false;
    std::vector<int64_t> shape_;
    DType dtype_ = DType::Float32;
};

}  // namespace msplat
