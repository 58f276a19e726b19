// dnn/core/fp8.hpp -- element types and dtype traits of the drop-in tensor.
//
// The reference instantiates tensor<> for the packed 4-value types
// __nv_fp8x4_e4m3 / __nv_fp8x4_e5m2 (dnn/core/tensor.cu:489-498, compiled
// only when __CUDA_FP8_TYPES_EXIST__); here each fp8 element is one byte
// holding an OCP OFP8 code, and the per-tensor scale lives with the tensor.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <type_traits>

#include "df_capi.h"

namespace dnn {

struct fp8_e4m3 {
    uint8_t bits = 0;
    constexpr fp8_e4m3() = default;
    constexpr explicit fp8_e4m3(uint8_t b) : bits(b) {}
    constexpr bool operator==(const fp8_e4m3& o) const { return bits == o.bits; }
    constexpr bool operator!=(const fp8_e4m3& o) const { return bits != o.bits; }
};
struct fp8_e5m2 {
    uint8_t bits = 0;
    constexpr fp8_e5m2() = default;
    constexpr explicit fp8_e5m2(uint8_t b) : bits(b) {}
    constexpr bool operator==(const fp8_e5m2& o) const { return bits == o.bits; }
    constexpr bool operator!=(const fp8_e5m2& o) const { return bits != o.bits; }
};
static_assert(sizeof(fp8_e4m3) == 1 && sizeof(fp8_e5m2) == 1, "fp8 elements are one byte");

using bfloat16 = __hip_bfloat16;

// The project's element-type enum: values 0-4 as the reference's
// DType (dnn/utils/onnx_loader.cuh:16-22), extended with the
// two fp8 formats; the same values as df_dtype in the C ABI.
enum class DType : uint8_t {
    Float32 = DF_DTYPE_FLOAT32,
    Half = DF_DTYPE_HALF,
    Int8 = DF_DTYPE_INT8,
    UInt8 = DF_DTYPE_UINT8,
    BFloat16 = DF_DTYPE_BFLOAT16,
    FP8E4M3 = DF_DTYPE_FP8E4M3,
    FP8E5M2 = DF_DTYPE_FP8E5M2,
};
static_assert((int)DType::Float32 == 0 && (int)DType::BFloat16 == 4 && (int)DType::FP8E4M3 == 5 &&
                  (int)DType::FP8E5M2 == 6,
              "enum values are part of the on-disk and C-ABI contract");

template <typename T> struct dtype_traits;
template <> struct dtype_traits<float> { static constexpr int value = DF_DTYPE_FLOAT32; static constexpr bool is_fp8 = false; };
template <> struct dtype_traits<__half> { static constexpr int value = DF_DTYPE_HALF; static constexpr bool is_fp8 = false; };
template <> struct dtype_traits<bfloat16> { static constexpr int value = DF_DTYPE_BFLOAT16; static constexpr bool is_fp8 = false; };
template <> struct dtype_traits<int8_t> { static constexpr int value = DF_DTYPE_INT8; static constexpr bool is_fp8 = false; };
template <> struct dtype_traits<uint8_t> { static constexpr int value = DF_DTYPE_UINT8; static constexpr bool is_fp8 = false; };
template <> struct dtype_traits<int> { static constexpr int value = DF_DTYPE_INT32; static constexpr bool is_fp8 = false; };
template <> struct dtype_traits<fp8_e4m3> {
    static constexpr int value = DF_DTYPE_FP8E4M3;
    static constexpr bool is_fp8 = true;
    static constexpr int fmt = DF_FMT_E4M3;
};
template <> struct dtype_traits<fp8_e5m2> {
    static constexpr int value = DF_DTYPE_FP8E5M2;
    static constexpr bool is_fp8 = true;
    static constexpr int fmt = DF_FMT_E5M2;
};

}  // namespace dnn
