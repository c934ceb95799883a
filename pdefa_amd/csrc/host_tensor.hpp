// Host tensors behind the EngineTensor handle: rank <= 8, 64-byte aligned,
// uninitialised on creation (as the reference's Tensor::empty,
// PDEFA1.0/src/core/tensor.cpp:68-80).
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <new>

namespace pdefa {

constexpr int kMaxNdim = 8;

// Page-locked host memory (defined by the device runtime): tensors created
// through the public API from this size up live there, so that a session's
// upload of them is a DMA transfer.  pinned_alloc returns nullptr when no
// HIP device is available or the allocation fails.
constexpr size_t kPinnedMinBytes = 256 * 1024;
void* pinned_alloc(size_t bytes);
void pinned_free(void* p);

// Public EngineDType codes (PDEFA1.0/include/engine/engine_c_api.h:53-62).
enum DT : int32_t { kF32 = 0, kF16 = 1, kBF16 = 2, kI8 = 3, kU8 = 4, kI32 = 5, kI64 = 6, kBool = 7 };

inline size_t dt_size(int32_t dt) {
    switch (dt) {
        case kF32: return 4;
        case kF16: return 2;
        case kBF16: return 2;
        case kI8: return 1;
        case kU8: return 1;
        case kI32: return 4;
        case kI64: return 8;
        case kBool: return 1;
        default: return 0;
    }
}

struct HostTensor {
    int32_t dtype = kF32;
    int32_t rank = 0;
    int64_t dims[kMaxNdim] = {0, 0, 0, 0, 0, 0, 0, 0};
    void* data = nullptr;
    size_t nbytes = 0;
    bool owns = false;
    bool pinned = false;  // data from pinned_alloc

    HostTensor() = default;
    HostTensor(const HostTensor&) = delete;
    HostTensor& operator=(const HostTensor&) = delete;
    HostTensor(HostTensor&& o) noexcept { *this = static_cast<HostTensor&&>(o); }
    HostTensor& operator=(HostTensor&& o) noexcept {
        if (this != &o) {
            release();
            dtype = o.dtype;
            rank = o.rank;
            std::memcpy(dims, o.dims, sizeof(dims));
            data = o.data;
            nbytes = o.nbytes;
            owns = o.owns;
            pinned = o.pinned;
            o.data = nullptr;
            o.nbytes = 0;
            o.owns = false;
            o.pinned = false;
        }
        return *this;
    }
    ~HostTensor() { release(); }

    void release() {
        if (owns && data) {
            if (pinned)
                pinned_free(data);
            else
                std::free(data);
        }
        data = nullptr;
        owns = false;
        pinned = false;
    }

    int64_t numel() const {
        int64_t n = 1;
        for (int i = 0; i < rank; ++i) n *= dims[i];
        return n;
    }
    int64_t dim(int i) const { return (i >= 0 && i < rank) ? dims[i] : 0; }
    float* f32() { return static_cast<float*>(data); }
    const float* f32() const { return static_cast<const float*>(data); }

    // Allocates (uninitialised).  Throws std::bad_alloc on failure.
    static HostTensor empty(const int64_t* shape, int32_t ndim, int32_t dtype) {
        HostTensor t;
        t.dtype = dtype;
        t.rank = ndim < 0 ? 0 : (ndim > kMaxNdim ? kMaxNdim : ndim);
        for (int i = 0; i < t.rank; ++i) t.dims[i] = shape[i];
        const int64_t n = t.numel();
        t.nbytes = n > 0 ? static_cast<size_t>(n) * dt_size(dtype) : 0;
        if (t.nbytes > 0) {
            const size_t alloc = (t.nbytes + 63) / 64 * 64;
            t.data = std::aligned_alloc(64, alloc);
            if (!t.data) throw std::bad_alloc();
            t.owns = true;
        }
        return t;
    }

    // empty(), in page-locked memory when the tensor is at least
    // kPinnedMinBytes and a device is there (tensors of the public API)
    static HostTensor empty_pinned(const int64_t* shape, int32_t ndim, int32_t dtype) {
        HostTensor t;
        t.dtype = dtype;
        t.rank = ndim < 0 ? 0 : (ndim > kMaxNdim ? kMaxNdim : ndim);
        for (int i = 0; i < t.rank; ++i) t.dims[i] = shape[i];
        const int64_t n = t.numel();
        const size_t nb = n > 0 ? static_cast<size_t>(n) * dt_size(dtype) : 0;
        if (nb >= kPinnedMinBytes) {
            if (void* p = pinned_alloc((nb + 63) / 64 * 64)) {
                t.nbytes = nb;
                t.data = p;
                t.owns = true;
                t.pinned = true;
                return t;
            }
        }
        return empty(shape, ndim, dtype);
    }

    HostTensor clone() const {
        HostTensor t = empty(dims, rank, dtype);
        if (nbytes) std::memcpy(t.data, data, nbytes);
        return t;
    }
};

}  // namespace pdefa
