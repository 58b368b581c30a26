// Tensor view of the Viper host API.
//
// DType values, Shape and Tensor follow the reference
// (include/viper/tensor.h:14-115): a Tensor is a non-owning view (data
// pointer, dtype, shape), row-major.  Device memory is owned by the caller.
// dtype_sizeof returns 1 for the packed quantized dtypes, as the reference
// does (src/viper/tensor.cpp:35-38); their byte size comes from
// quant::packed_bytes.
#pragma once

#include <array>
#include <initializer_list>

#include "viper/common.h"

namespace viper {

enum class DType : int {
    FP32 = 0,
    BF16 = 1,
    FP16 = 2,
    INT8 = 3,
    UINT8 = 4,
    INT32 = 5,
    UINT32 = 6,
    Q4_G64 = 100,
    Q5_G64 = 101,
    Q6_G64 = 102,
    W8_G32 = 103,
};

const char* dtype_name(DType d) noexcept;
usize dtype_sizeof(DType d) noexcept;

class Shape {
  public:
    using Dim = i64;
    static constexpr usize kMaxDims = 8;

    Shape() = default;
    Shape(std::initializer_list<Dim> dims) {
        for (auto d : dims) {
            if (rank_ == kMaxDims) break;
            dims_[rank_++] = d;
        }
    }
    Shape(const Dim* dims, usize n) {
        for (usize i = 0; i < n && i < kMaxDims; ++i) dims_[rank_++] = dims[i];
    }

    Dim operator[](usize i) const noexcept { return dims_[i]; }
    Dim& operator[](usize i) noexcept { return dims_[i]; }
    usize rank() const noexcept { return rank_; }
    Dim dim(usize i) const noexcept { return dims_[i]; }
    i64 numel() const noexcept {
        i64 n = 1;
        for (usize i = 0; i < rank_; ++i) n *= dims_[i];
        return n;
    }
    bool operator==(const Shape& o) const noexcept {
        if (rank_ != o.rank_) return false;
        for (usize i = 0; i < rank_; ++i)
            if (dims_[i] != o.dims_[i]) return false;
        return true;
    }
    bool operator!=(const Shape& o) const noexcept { return !(*this == o); }

  private:
    std::array<Dim, kMaxDims> dims_{};
    usize rank_ = 0;
};

class Tensor {
  public:
    Tensor() = default;
    Tensor(void* data, DType dtype, Shape shape) : data_(data), dtype_(dtype), shape_(shape) {}

    void* data() const noexcept { return data_; }
    DType dtype() const noexcept { return dtype_; }
    const Shape& shape() const noexcept { return shape_; }
    i64 numel() const noexcept { return shape_.numel(); }
    usize nbytes() const noexcept { return static_cast<usize>(numel()) * dtype_sizeof(dtype_); }

    template <typename T>
    T* data_as() const noexcept {
        return reinterpret_cast<T*>(data_);
    }

  private:
    void* data_ = nullptr;
    DType dtype_ = DType::FP32;
    Shape shape_;
};

}  // namespace viper
