// tensor_ops.hip -- library plumbing (error string, version) and the small
// elementwise kernels behind dnn::tensor: fill, add, equal / approx-equal
// masks (dnn/core/tensor.cu:18-52 in the reference).  These are not on the
// fp8 hot path; they exist so the C++ drop-in tensor does its device work
// through the C ABI like everything else.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "df_common.hpp"

namespace dfk {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

// Every entry point starts here: besides the message, this resets the HIP
// runtime's per-thread last error, so that launch_status() reports only
// what this call's launches raised, not a failed runtime call the caller
// made earlier (a sticky device fault is still reported, by every call).
void clear_error() {
    g_last_error.clear();
    (void)hipGetLastError();
}

int launch_status(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
        return DF_ERR_HIP;
    }
    return DF_OK;
}

int device_cu_count() {
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (dev < 0 || dev >= 64) return 0;
    int n = __atomic_load_n(&cached[dev], __ATOMIC_RELAXED);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        __atomic_store_n(&cached[dev], n, __ATOMIC_RELAXED);
    }
    return n;
}

constexpr int kThreads = 256;

template <typename T>
__global__ __launch_bounds__(kThreads) void fill_kernel(T* __restrict__ p, int64_t n, T v) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) p[i] = v;
}

// element loaders/storers by dtype, in fp32 for floating types
template <int DT> struct Elem;
template <> struct Elem<DF_DTYPE_FLOAT32> {
    using T = float;
    static __device__ float ld(T v) { return v; }
    static __device__ T st(float f) { return f; }
};
template <> struct Elem<DF_DTYPE_HALF> {
    using T = uint16_t;
    static __device__ float ld(T v) { return f16_to_f32(v); }
    static __device__ T st(float f) { return (T)f32_to_f16_rne(f); }
};
template <> struct Elem<DF_DTYPE_INT8> {  // input side only (exact widening)
    using T = int8_t;
    static __device__ float ld(T v) { return (float)v; }
};
template <> struct Elem<DF_DTYPE_BFLOAT16> {
    using T = uint16_t;
    static __device__ float ld(T v) { return bf16_to_f32(v); }
    static __device__ T st(float f) { return (T)f32_to_bf16_rne(f); }
};

// floating add in fp32 then round; integer add wraps like the reference's
// a[idx] + b[idx] on the element type.
template <int DT>
__global__ __launch_bounds__(kThreads) void add_float_kernel(const typename Elem<DT>::T* a,
                                                              const typename Elem<DT>::T* b,
                                                              typename Elem<DT>::T* out, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
        out[i] = Elem<DT>::st(Elem<DT>::ld(a[i]) + Elem<DT>::ld(b[i]));
}

template <typename T>
__global__ __launch_bounds__(kThreads) void add_int_kernel(const T* a, const T* b, T* out, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
        out[i] = (T)(a[i] + b[i]);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void equal_kernel(const T* a, const T* b, uint8_t* m, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
        m[i] = a[i] == b[i] ? 1 : 0;
}

template <int DT>
__global__ __launch_bounds__(kThreads) void approx_float_kernel(const typename Elem<DT>::T* a,
                                                                 const typename Elem<DT>::T* b,
                                                                 uint8_t* m, int64_t n, float atol) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
        m[i] = fabsf(Elem<DT>::ld(a[i]) - Elem<DT>::ld(b[i])) <= atol ? 1 : 0;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void approx_int_kernel(const T* a, const T* b, uint8_t* m,
                                                               int64_t n, float atol) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
        m[i] = fabsf((float)a[i] - (float)b[i]) <= atol ? 1 : 0;
}

template <int DI, int DO>
__global__ __launch_bounds__(kThreads) void convert_kernel(const typename Elem<DI>::T* __restrict__ in,
                                                            typename Elem<DO>::T* __restrict__ out, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
        out[i] = Elem<DO>::st(Elem<DI>::ld(in[i]));
}

static int blocks_for(int64_t n) {
    int64_t b = (n + kThreads - 1) / kThreads;
    if (b > 4096) b = 4096;
    return b < 1 ? 1 : (int)b;
}

}  // namespace dfk

using namespace dfk;

extern "C" const char* df_last_error_string(void) { return g_last_error.c_str(); }
extern "C" int df_version(void) { return 100; }

extern "C" int df_device_arch_ok(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
    return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

extern "C" int df_fill(void* dst, int64_t n, int elem_bytes, const void* value_host, void* stream) {
    clear_error();
    DF_CHECK(n >= 0, DF_ERR_INVALID, "df_fill: n < 0");
    if (n == 0) return DF_OK;
    DF_CHECK(dst && value_host, DF_ERR_INVALID, "df_fill: NULL pointer");
    hipStream_t st = as_stream(stream);
    const int blocks = blocks_for(n);
    switch (elem_bytes) {
        case 1: fill_kernel<uint8_t><<<blocks, kThreads, 0, st>>>((uint8_t*)dst, n, *(const uint8_t*)value_host); break;
        case 2: fill_kernel<uint16_t><<<blocks, kThreads, 0, st>>>((uint16_t*)dst, n, *(const uint16_t*)value_host); break;
        case 4: fill_kernel<uint32_t><<<blocks, kThreads, 0, st>>>((uint32_t*)dst, n, *(const uint32_t*)value_host); break;
        default: DF_CHECK(false, DF_ERR_UNSUPPORTED, "df_fill: elem_bytes %d", elem_bytes);
    }
    return launch_status("df_fill");
}

extern "C" int df_convert(int in_dtype, const void* in, int out_dtype, void* out, int64_t n, void* stream) {
    clear_error();
    DF_CHECK(n >= 0, DF_ERR_INVALID, "df_convert: n < 0");
    if (n == 0) return DF_OK;
    DF_CHECK(in && out, DF_ERR_INVALID, "df_convert: NULL pointer");
    hipStream_t st = as_stream(stream);
    const int g = blocks_for(n);
#define DF_CVT(I, O)                                                                                  \
    if (in_dtype == I && out_dtype == O) {                                                            \
        convert_kernel<I, O><<<g, kThreads, 0, st>>>((const typename Elem<I>::T*)in, (typename Elem<O>::T*)out, n); \
        return launch_status("df_convert");                                                           \
    }
    DF_CVT(DF_DTYPE_FLOAT32, DF_DTYPE_FLOAT32)
    DF_CVT(DF_DTYPE_FLOAT32, DF_DTYPE_BFLOAT16)
    DF_CVT(DF_DTYPE_FLOAT32, DF_DTYPE_HALF)
    DF_CVT(DF_DTYPE_BFLOAT16, DF_DTYPE_FLOAT32)
    DF_CVT(DF_DTYPE_BFLOAT16, DF_DTYPE_HALF)
    DF_CVT(DF_DTYPE_HALF, DF_DTYPE_FLOAT32)
    DF_CVT(DF_DTYPE_INT8, DF_DTYPE_FLOAT32)
    DF_CVT(DF_DTYPE_INT8, DF_DTYPE_HALF)
#undef DF_CVT
    DF_CHECK(false, DF_ERR_UNSUPPORTED, "df_convert: %d -> %d not supported", in_dtype, out_dtype);
}

extern "C" int df_add(int dtype, const void* a, const void* b, void* out, int64_t n, void* stream) {
    clear_error();
    DF_CHECK(n >= 0, DF_ERR_INVALID, "df_add: n < 0");
    if (n == 0) return DF_OK;
    DF_CHECK(a && b && out, DF_ERR_INVALID, "df_add: NULL pointer");
    hipStream_t st = as_stream(stream);
    const int g = blocks_for(n);
    switch (dtype) {
        case DF_DTYPE_FLOAT32: add_float_kernel<DF_DTYPE_FLOAT32><<<g, kThreads, 0, st>>>((const float*)a, (const float*)b, (float*)out, n); break;
        case DF_DTYPE_HALF: add_float_kernel<DF_DTYPE_HALF><<<g, kThreads, 0, st>>>((const uint16_t*)a, (const uint16_t*)b, (uint16_t*)out, n); break;
        case DF_DTYPE_BFLOAT16: add_float_kernel<DF_DTYPE_BFLOAT16><<<g, kThreads, 0, st>>>((const uint16_t*)a, (const uint16_t*)b, (uint16_t*)out, n); break;
        case DF_DTYPE_INT8: add_int_kernel<int8_t><<<g, kThreads, 0, st>>>((const int8_t*)a, (const int8_t*)b, (int8_t*)out, n); break;
        case DF_DTYPE_UINT8: add_int_kernel<uint8_t><<<g, kThreads, 0, st>>>((const uint8_t*)a, (const uint8_t*)b, (uint8_t*)out, n); break;
        case DF_DTYPE_INT32: add_int_kernel<int32_t><<<g, kThreads, 0, st>>>((const int32_t*)a, (const int32_t*)b, (int32_t*)out, n); break;
        default: DF_CHECK(false, DF_ERR_UNSUPPORTED, "df_add: dtype %d not supported", dtype);
    }
    return launch_status("df_add");
}

extern "C" int df_equal_mask(int dtype, const void* a, const void* b, uint8_t* mask, int64_t n,
                             void* stream) {
    clear_error();
    DF_CHECK(n >= 0, DF_ERR_INVALID, "df_equal_mask: n < 0");
    if (n == 0) return DF_OK;
    DF_CHECK(a && b && mask, DF_ERR_INVALID, "df_equal_mask: NULL pointer");
    hipStream_t st = as_stream(stream);
    const int g = blocks_for(n);
    switch (dtype) {
        case DF_DTYPE_FLOAT32:
        case DF_DTYPE_INT32: equal_kernel<uint32_t><<<g, kThreads, 0, st>>>((const uint32_t*)a, (const uint32_t*)b, mask, n); break;
        case DF_DTYPE_HALF:
        case DF_DTYPE_BFLOAT16: equal_kernel<uint16_t><<<g, kThreads, 0, st>>>((const uint16_t*)a, (const uint16_t*)b, mask, n); break;
        case DF_DTYPE_INT8:
        case DF_DTYPE_UINT8:
        case DF_DTYPE_FP8E4M3:
        case DF_DTYPE_FP8E5M2: equal_kernel<uint8_t><<<g, kThreads, 0, st>>>((const uint8_t*)a, (const uint8_t*)b, mask, n); break;
        default: DF_CHECK(false, DF_ERR_UNSUPPORTED, "df_equal_mask: dtype %d not supported", dtype);
    }
    return launch_status("df_equal_mask");
}

extern "C" int df_approx_equal_mask(int dtype, const void* a, const void* b, uint8_t* mask, int64_t n,
                                    float atol, void* stream) {
    clear_error();
    DF_CHECK(n >= 0, DF_ERR_INVALID, "df_approx_equal_mask: n < 0");
    if (n == 0) return DF_OK;
    DF_CHECK(a && b && mask, DF_ERR_INVALID, "df_approx_equal_mask: NULL pointer");
    hipStream_t st = as_stream(stream);
    const int g = blocks_for(n);
    switch (dtype) {
        case DF_DTYPE_FLOAT32: approx_float_kernel<DF_DTYPE_FLOAT32><<<g, kThreads, 0, st>>>((const float*)a, (const float*)b, mask, n, atol); break;
        case DF_DTYPE_HALF: approx_float_kernel<DF_DTYPE_HALF><<<g, kThreads, 0, st>>>((const uint16_t*)a, (const uint16_t*)b, mask, n, atol); break;
        case DF_DTYPE_BFLOAT16: approx_float_kernel<DF_DTYPE_BFLOAT16><<<g, kThreads, 0, st>>>((const uint16_t*)a, (const uint16_t*)b, mask, n, atol); break;
        case DF_DTYPE_INT8: approx_int_kernel<int8_t><<<g, kThreads, 0, st>>>((const int8_t*)a, (const int8_t*)b, mask, n, atol); break;
        case DF_DTYPE_UINT8: approx_int_kernel<uint8_t><<<g, kThreads, 0, st>>>((const uint8_t*)a, (const uint8_t*)b, mask, n, atol); break;
        case DF_DTYPE_INT32: approx_int_kernel<int32_t><<<g, kThreads, 0, st>>>((const int32_t*)a, (const int32_t*)b, mask, n, atol); break;
        default: DF_CHECK(false, DF_ERR_UNSUPPORTED, "df_approx_equal_mask: dtype %d not supported", dtype);
    }
    return launch_status("df_approx_equal_mask");
}
