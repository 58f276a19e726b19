// dnn/utils/common.hpp -- error plumbing of the C++ drop-in.
//
// Mirrors dnn/utils/common.cuh:20-35 of the reference (HIP runtime errors and
// C-ABI status codes become std::runtime_error with file:line), and keeps the
// reference's macro names as aliases so callers compile unchanged.
#pragma once

#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>
#include <vector>

#include "df_capi.h"

namespace dnn {
template <typename TT>
struct tensor;
}

namespace dnn::utils {

// Gradient clipping by global L2 norm, as declared at dnn/utils/common.cuh:
// 116-119 (defined clip_grad_norm.cu:31-62): when the norm over every
// element of every tensor exceeds max_norm, each element is multiplied by
// max_norm / norm.  Provided for T = float.  The norm is computed and
// compared on the device (the reference downloads each gradient and sums on
// the host), so the call only enqueues work on Hip::stream().
template <typename T>
void clip_grad_norm(std::vector<tensor<T>*>& gradients, T max_norm);

inline void check_hip_error(hipError_t error, const char* file, int line) {
    if (error != hipSuccess) {
        (void)hipGetLastError();  // the error is reported here, not by the next call
        throw std::runtime_error(std::string("HIP error at ") + file + ":" + std::to_string(line) + ": " +
                                 hipGetErrorString(error));
    }
}

inline void check_hip_error(const char* file, int line) { check_hip_error(hipGetLastError(), file, line); }

// A negative df_status from the C ABI, with the library's message.
inline void check_df_status(int status, const char* what, const char* file, int line) {
    if (status != DF_OK)
        throw std::runtime_error(std::string(what) + " failed (status " + std::to_string(status) + ") at " + file +
                                 ":" + std::to_string(line) + ": " + df_last_error_string());
}

}  // namespace dnn::utils

#define CHECK_HIP_EX(call) ::dnn::utils::check_hip_error((call), __FILE__, __LINE__)
#define THROW_HIP_EX() ::dnn::utils::check_hip_error(__FILE__, __LINE__)
#define CHECK_DF_EX(call) ::dnn::utils::check_df_status((call), #call, __FILE__, __LINE__)
// reference spellings (dnn/utils/common.cuh:34-35)
#define CHECK_CUDA_EX(call) CHECK_HIP_EX(call)
#define THROW_CUDA_EX() THROW_HIP_EX()
