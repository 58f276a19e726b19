// dnn/core/tensor.hpp -- device tensor of the drop-in (namespace dnn).
//
// Same public contract as the reference's tensor<TT> (dnn/core/tensor.cuh:
// 23-149): a move-only owner of one contiguous row-major device buffer with
// an int shape; upload/download are synchronous; fill, +=, +, ==, equals,
// approx_equal, clone, reshape, save/load behave as there.  Element types:
// float, __half, bfloat16, int8_t, uint8_t, int, and the one-byte
// fp8_e4m3 / fp8_e5m2, whose tensors also carry a per-tensor scale (one
// float on the device) so that value = decode(code) * scale.
//
// Device work goes through the C ABI (include/df_capi.h) on Hip::stream().
// narrow/slice/transpose/permute are not part of this build (they are not
// on the fp8 Linear path).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <iostream>
#include <string>
#include <vector>

#include "dnn/core/fp8.hpp"

namespace dnn {

template <typename TT>
struct tensor {
protected:
    std::vector<int> shape_;
    TT* data_ = nullptr;
    int total_size_ = 0;
    float* scale_ = nullptr;  // fp8 tensors only: device float, value = code * scale

public:
    explicit tensor(const std::vector<int>& shape);
    virtual ~tensor();

    virtual void upload(const TT* host_data);
    virtual void download(TT* host_data) const;

    TT* data() { return data_; }
    const TT* data() const { return data_; }
    const std::vector<int>& shape() const { return shape_; }
    int size() const { return total_size_; }
    int size(int dim) const;

    tensor<TT>& reshape(const std::vector<int>& new_shape);
    tensor<TT>& fill(TT value);
    tensor<TT>& zero();

    tensor(const tensor&) = delete;
    tensor& operator=(const tensor&) = delete;
    tensor(tensor&& other) noexcept;
    tensor& operator=(tensor&& other) noexcept;

    tensor<TT> clone() const;
    tensor<TT>& operator+=(const tensor<TT>& other);
    tensor<uint8_t> operator==(const tensor<TT>& other) const;
    bool equals(const tensor<TT>& other) const;
    bool approx_equal(const tensor<TT>& other, float atol = 1e-5f) const;
    std::string to_string() const;

    // fp8 tensors: the per-tensor scale (device pointer / host value)
    float* scale_data() { return scale_; }
    const float* scale_data() const { return scale_; }
    float scale() const;
    void set_scale(float s);

    // Serialisation: int ndim, int dims[ndim], raw elements (the reference's
    // layout, tensor.cuh:104-125).  fp8 tensors write a tagged record (a
    // negative tag, the DType value, then that layout and the float scale);
    // float and bfloat16 tensors also load such a record, dequantized.
    void save(std::ostream& out) const;
    void load(std::istream& in);
};

template <typename TT>
tensor<TT> operator+(const tensor<TT>& a, const tensor<TT>& b);

// ---- fp8 conversions (the dnn/core quantize / dequantize of this path) ----
// quantize: per-tensor absmax scale s = absmax / FMAX, codes = sat_rne(x / s)
// (include/df_capi.h states the full contract); dequantize: code * s.
template <typename Q, typename T>
tensor<Q> quantize(const tensor<T>& x);
template <typename T, typename Q>
tensor<T> dequantize(const tensor<Q>& q);

using tensorf = tensor<float>;
using tensorh = tensor<__half>;
using tensorbf = tensor<bfloat16>;
using tensori = tensor<int>;
using tensori8 = tensor<int8_t>;
using tensoru8 = tensor<uint8_t>;
using tensorf8e4m3 = tensor<fp8_e4m3>;
using tensorf8e5m2 = tensor<fp8_e5m2>;

}  // namespace dnn
