#pragma once
// ESTensor -- the minimal device tensor the ES* layer uses where the reference uses
// mx::array: a device pointer with shape and element strides, optionally owning its
// allocation (shared, so views keep the buffer alive like MLX's refcounted arrays).
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <vector>

namespace es {

enum class Dtype { bf16, f32, i32, u8 };

inline size_t dtypeSize(Dtype d) {
    switch (d) {
        case Dtype::bf16: return 2;
        case Dtype::f32: return 4;
        case Dtype::i32: return 4;
        default: return 1;
    }
}

struct Tensor {
    std::shared_ptr<void> storage;  // owner of the device allocation (null for borrowed data)
    void *data = nullptr;           // first element
    std::vector<int64_t> shape, strides;
    Dtype dtype = Dtype::bf16;
    int device = 0;

    int dim() const { return (int) shape.size(); }
    int64_t size(int axis) const { return shape.at(axis < 0 ? axis + dim() : axis); }
    int64_t numel() const {
        int64_t n = 1;
        for (int64_t s : shape) n *= s;
        return n;
    }
    bool defined() const { return data != nullptr; }
    bool contiguous() const {
        int64_t expect = 1;
        for (int i = dim() - 1; i >= 0; --i) {
            if (shape[i] != 1 && strides[i] != expect) return false;
            expect *= shape[i];
        }
        return true;
    }
    size_t nbytes() const { return (size_t) numel() * dtypeSize(dtype); }

    // Contiguous strides for `shape`.
    static std::vector<int64_t> denseStrides(const std::vector<int64_t> &shape) {
        std::vector<int64_t> st(shape.size(), 1);
        for (int i = (int) shape.size() - 2; i >= 0; --i) st[i] = st[i + 1] * shape[i + 1];
        return st;
    }

    // New device allocation (uninitialised) on the current device, sized in whole 4-byte
    // words so that a word-wise fill of the tensor stays inside it.
    static Tensor empty(const std::vector<int64_t> &shape, Dtype dtype) {
        Tensor t;
        t.shape = shape;
        t.strides = denseStrides(shape);
        t.dtype = dtype;
        if (hipGetDevice(&t.device) != hipSuccess) throw std::runtime_error("ESTensor: hipGetDevice failed");
        void *p = nullptr;
        const size_t bytes = t.nbytes() ? (t.nbytes() + 3) / 4 * 4 : 16;
        if (hipMalloc(&p, bytes) != hipSuccess) throw std::runtime_error("ESTensor: hipMalloc failed");
        t.storage = std::shared_ptr<void>(p, [](void *q) { (void) hipFree(q); });
        t.data = p;
        return t;
    }

    // Borrowed view of caller-owned memory.
    static Tensor wrap(void *ptr, const std::vector<int64_t> &shape, Dtype dtype,
                       std::vector<int64_t> strides = {}) {
        Tensor t;
        t.data = ptr;
        t.shape = shape;
        t.strides = strides.empty() ? denseStrides(shape) : strides;
        t.dtype = dtype;
        (void) hipGetDevice(&t.device);
        return t;
    }

    // View of [begin, end) along `axis` (shares storage).
    Tensor slice(int axis, int64_t begin, int64_t end) const {
        if (axis < 0) axis += dim();
        if (begin < 0 || end > shape.at(axis) || begin > end) throw std::invalid_argument("ESTensor::slice out of range");
        Tensor t = *this;
        t.data = static_cast<char *>(data) + begin * strides[axis] * (int64_t) dtypeSize(dtype);
        t.shape[axis] = end - begin;
        return t;
    }
};

}  // namespace es
