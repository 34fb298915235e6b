// mtensor.hpp -- MTensor: shape/dtype metadata over a device (hipMalloc) or
// host allocation, with the reference's API names (core/include/
// metal_tensor.hpp:36-143: numel/size/ndim/shape/dtype/nbytes/data_ptr/
// data<T>/zero/cpu/reset/stride0/view).
//
// Differences that follow from discrete HBM instead of Apple unified memory:
//  - data_ptr() of a GPU tensor is a device pointer; read it on the host
//    through cpu() (a synchronous copy) or copy_to_host();
//  - storage is reference counted, so copies and view(n) keep the buffer
//    alive (the reference's views are non-owning, metal_tensor.hpp:121-124).
#pragma once

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "msplat_engine.h"

enum class DType : uint8_t {
    Float32,
    Int32,
    Int64,
    UInt8,
    Float64,
};

inline size_t dtypeSize(DType dt) {
    switch (dt) {
        case DType::Float32: return 4;
        case DType::Int32: return 4;
        case DType::Int64: return 8;
        case DType::UInt8: return 1;
        case DType::Float64: return 8;
    }
    return 4;
}

class MTensor {
public:
    MTensor() = default;

    // Host allocation (the reference's CPU constructor).
    MTensor(std::vector<int64_t> shape, DType dtype) : _shape(std::move(shape)), _dtype(dtype) {
        _numel = count(_shape);
        auto st = std::make_shared<Storage>();
        st->host.resize(std::max<size_t>(nbytes(), 1));
        st->bytes = st->host.size();
        _st = st;
    }

    static MTensor device(std::vector<int64_t> shape, DType dtype) {
        MTensor t;
        t._shape = std::move(shape);
        t._dtype = dtype;
        t._numel = count(t._shape);
        auto st = std::make_shared<Storage>();
        st->bytes = std::max<size_t>(t.nbytes(), 16);
        st->dev = msplat_hip_alloc(st->bytes);
        if (!st->dev) throw std::runtime_error(std::string("device allocation failed: ") + msplat_hip_last_error());
        t._st = st;
        return t;
    }

    // Non-owning wrapper around an engine-owned device buffer (the
    // msplat_last_* accessors); valid until the engine reallocates it.
    static MTensor wrap_device(void *ptr, std::vector<int64_t> shape, DType dtype) {
        MTensor t;
        t._shape = std::move(shape);
        t._dtype = dtype;
        t._numel = count(t._shape);
        auto st = std::make_shared<Storage>();
        st->dev = ptr;
        st->owned = false;
        st->bytes = t.nbytes();
        t._st = st;
        return t;
    }

    bool defined() const { return (bool)_st; }
    bool isGpu() const { return _st && _st->dev; }

    int64_t numel() const { return _numel; }
    int64_t size(int dim) const {
        if (dim < 0) dim += (int)_shape.size();
        return _shape.at(dim);
    }
    int ndim() const { return (int)_shape.size(); }
    const std::vector<int64_t> &shape() const { return _shape; }
    DType dtype() const { return _dtype; }
    size_t elementSize() const { return dtypeSize(_dtype); }
    size_t nbytes() const { return (size_t)_numel * dtypeSize(_dtype); }

    void *data_ptr() {
        if (!_st) return nullptr;
        return _st->dev ? _st->dev : (void *)_st->host.data();
    }
    const void *data_ptr() const { return const_cast<MTensor *>(this)->data_ptr(); }
    template <typename T>
    T *data() {
        return static_cast<T *>(data_ptr());
    }
    template <typename T>
    const T *data() const {
        return static_cast<const T *>(data_ptr());
    }

    void zero() {
        if (!_st) return;
        if (_st->dev)
            check(msplat_hip_memset(_st->dev, 0, nbytes()));
        else
            std::memset(data_ptr(), 0, nbytes());
    }

    // Synchronous copy to host memory.
    MTensor cpu() const {
        MTensor out(_shape, _dtype);
        copy_to_host(out.data_ptr());
        return out;
    }
    // Copy to a new device tensor (host or device source).
    MTensor gpu() const {
        MTensor out = MTensor::device(_shape, _dtype);
        if (nbytes() == 0) return out;
        if (isGpu())
            check(msplat_hip_copy(out.data_ptr(), data_ptr(), nbytes()));
        else
            check(msplat_hip_upload(out.data_ptr(), data_ptr(), nbytes()));
        return out;
    }
    void copy_to_host(void *dst) const {
        if (!_st || nbytes() == 0) return;
        if (_st->dev)
            check(msplat_hip_download(dst, data_ptr(), nbytes()));
        else
            std::memcpy(dst, data_ptr(), nbytes());
    }
    void copy_from_host(const void *src, size_t bytes) {
        if (bytes > nbytes()) throw std::runtime_error("copy_from_host: size exceeds tensor");
        if (!bytes) return;
        if (isGpu())
            check(msplat_hip_upload(data_ptr(), src, bytes));
        else
            std::memcpy(data_ptr(), src, bytes);
    }

    void reset() {
        _st.reset();
        _shape.clear();
        _numel = 0;
    }

    int64_t stride0() const {
        if (_shape.size() <= 1) return 1;
        int64_t s = 1;
        for (size_t i = 1; i < _shape.size(); i++) s *= _shape[i];
        return s;
    }

    // The first n rows along dim 0; shares (and keeps alive) the storage.
    MTensor view(int64_t n) const {
        MTensor v = *this;
        v._shape[0] = n;
        v._numel = n * stride0();
        return v;
    }

private:
    struct Storage {
        void *dev = nullptr;
        bool owned = true;
        std::vector<uint8_t> host;
        size_t bytes = 0;
        ~Storage() {
            if (dev && owned) msplat_hip_free(dev);
        }
    };

    static int64_t count(const std::vector<int64_t> &s) {
        int64_t n = 1;
        for (auto d : s) n *= d;
        return n;
    }
    static void check(int rc) {
        if (rc != MSPLAT_OK) throw std::runtime_error(std::string("msplat engine: ") + msplat_hip_last_error());
    }

    std::shared_ptr<Storage> _st;
    std::vector<int64_t> _shape;
    DType _dtype = DType::Float32;
    int64_t _numel = 0;
};
