// optim.hip -- consumer side of the fp32 gradients: global-norm clipping and
// the Adam update, over lists of fp32 tensors (gfx950).
//
// Reference: dnn/utils/clip_grad_norm.cu:31-67 (norm over every gradient,
// then grad *= max_norm / norm when norm > max_norm) and
// dnn/optimizers/adam_optimizer.cu:11-30,83-109 (float path of
// adam_update_kernel, one launch per parameter tensor).
//
// Design:
//  - One launch covers up to kNormList (norm, clip) or kAdamList (Adam)
//    tensors: their pointers and sizes travel in the kernel arguments and
//    each block finds its tensor by a binary search of the first-block table
//    (uniform, scalar loads).  A block owns kChunk consecutive elements of
//    one tensor: 16-byte loads, kVec of them in flight per thread.
//  - The norm is computed on the device (the reference downloads every
//    gradient and sums on the host, clip_grad_norm.cu:38-39): squares are
//    formed in binary32 as in the reference, accumulated in binary64 per
//    thread, folded per block, and one block folds the block partials in a
//    fixed order.  The result is deterministic run to run.
//  - Whether to clip is decided on the device from the stored norm, so
//    clipping and the Adam step need no host synchronisation; the Adam
//    kernel can apply the clip factor itself, which saves the in-place
//    rewrite of every gradient.
//  - Every binary32 operation is the one written in the reference's float
//    path, each rounded (no contraction into fused multiply-adds), with
//    IEEE division and square root.
#include <hip/hip_runtime.h>

#include <math.h>

#include <vector>

#include "df_common.hpp"

// Rounding of every operation as written: no fused multiply-adds.
#pragma clang fp contract(off)

namespace dfk {

constexpr int kOThreads = 256;
constexpr int kVec = 8;                                        // float4 per thread per block
constexpr int64_t kChunk = (int64_t)kOThreads * 4 * kVec;     // 8192 elements per block
constexpr int kNormList = 64;
constexpr int kAdamList = 48;

struct NormList {
    float* ptr[kNormList];
    int64_t n[kNormList];
    int first[kNormList + 1];  // first block of each tensor; first[count] = blocks
    int count;
};

struct AdamList {
    float* p[kAdamList];
    const float* g[kAdamList];
    float* m[kAdamList];
    float* v[kAdamList];
    int64_t n[kAdamList];
    int first[kAdamList + 1];
    int idx[kAdamList];  // position in the caller's list (for the absmax output)
    int count;
};

struct AdamHyper {
    float lr, b1, b2, omb1, omb2, eps, wd;
    float bc1, bc2;    // 1 - beta^t, formed on the host
    float max_norm;    // used when a norm pointer is given
};

// tensor that owns block b: the last t with first[t] <= b
static __device__ __forceinline__ int owner(const int* first, int count, int b) {
    int lo = 0, hi = count - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (first[mid] <= b) lo = mid; else hi = mid - 1;
    }
    return lo;
}

static __device__ __forceinline__ double block_sum_f64(double s) {
    __shared__ double red[kOThreads / 64];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 1; w < kOThreads / 64; ++w) s += red[w];
    }
    return s;  // valid in thread 0
}

static __device__ __forceinline__ double sq(float x) { return (double)(x * x); }

// Stage 1 of the norm: one binary64 partial per block of kNormSub chunks
// (fewer partials for the single-block stage 2 to fold).
constexpr int kNormSub = 4;
constexpr int64_t kNormChunk = kChunk * kNormSub;

__global__ __launch_bounds__(kOThreads) void sumsq_kernel(const NormList L, double* __restrict__ partial,
                                                          int part0) {
    const int b = blockIdx.x;
    const int t = owner(L.first, L.count, b);
    const float* x = L.ptr[t];
    const int64_t n = L.n[t];
    double acc = 0.0;
    for (int sub = 0; sub < kNormSub; ++sub) {
        const int64_t base = (int64_t)(b - L.first[t]) * kNormChunk + sub * kChunk;
        if (base + kChunk <= n) {
            const f32x4* xv = reinterpret_cast<const f32x4*>(x + base);
            f32x4 r[kVec];
#pragma unroll
            for (int k = 0; k < kVec; ++k) r[k] = __builtin_nontemporal_load(xv + k * kOThreads + threadIdx.x);
#pragma unroll
            for (int k = 0; k < kVec; ++k) acc += sq(r[k].x) + sq(r[k].y) + sq(r[k].z) + sq(r[k].w);
        } else {
            for (int64_t i = base + threadIdx.x; i < n; i += kOThreads) acc += sq(x[i]);
            break;
        }
    }
    acc = block_sum_f64(acc);
    if (threadIdx.x == 0) partial[part0 + b] = acc;
}

// Stage 2: fixed-order fold of every partial; norm = RN32(sqrt(sum)).
// A GPT-2 XL sized list leaves ~180K partials: each thread keeps kFold
// independent loads in flight (a single dependent chain per thread made this
// one-block pass latency-bound).
constexpr int kFold = 8;
__global__ __launch_bounds__(kOThreads) void norm_finalize_kernel(const double* __restrict__ partial, int nparts,
                                                                  float* __restrict__ norm_out) {
    double acc[kFold];
#pragma unroll
    for (int j = 0; j < kFold; ++j) acc[j] = 0.0;
    int i = threadIdx.x;
    for (; i + (kFold - 1) * kOThreads < nparts; i += kFold * kOThreads) {
#pragma unroll
        for (int j = 0; j < kFold; ++j) acc[j] += partial[i + j * kOThreads];
    }
    for (; i < nparts; i += kOThreads) acc[0] += partial[i];
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < kFold; ++j) s += acc[j];
    s = block_sum_f64(s);
    if (threadIdx.x == 0) norm_out[0] = (float)sqrt(s);
}

// In-place clip: grad = grad * (max_norm / norm) when norm > max_norm
// (clip_grad_norm.cu:18 and :56); a NaN norm compares false and clips nothing.
__global__ __launch_bounds__(kOThreads) void clip_kernel(const NormList L, const float* __restrict__ norm,
                                                         float max_norm) {
    const float nv = norm[0];
    if (!(nv > max_norm)) return;
    const float f = max_norm / nv;
    const int b = blockIdx.x;
    const int t = owner(L.first, L.count, b);
    float* x = L.ptr[t];
    const int64_t n = L.n[t];
    const int64_t base = (int64_t)(b - L.first[t]) * kChunk;
    if (base + kChunk <= n) {
        f32x4* xv = reinterpret_cast<f32x4*>(x + base);
        f32x4 r[kVec];
#pragma unroll
        for (int k = 0; k < kVec; ++k) r[k] = __builtin_nontemporal_load(xv + k * kOThreads + threadIdx.x);
#pragma unroll
        for (int k = 0; k < kVec; ++k) {
            r[k].x = r[k].x * f; r[k].y = r[k].y * f; r[k].z = r[k].z * f; r[k].w = r[k].w * f;
            xv[k * kOThreads + threadIdx.x] = r[k];
        }
    } else {
        for (int64_t i = base + threadIdx.x; i < n; i += kOThreads) x[i] = x[i] * f;
    }
}

// adam_optimizer.cu:24-30, float path, one element:
//   g = grad + wd * p;  m = b1*m + (1-b1)*g;  v = b2*v + (1-b2)*g*g;
//   m_hat = m / (1 - b1^t);  v_hat = v / (1 - b2^t);
//   p = p - lr * m_hat / (sqrt(v_hat) + eps)
// with grad first multiplied by the clip factor f (1 when not clipping).
static __device__ __forceinline__ void adam1(float& p, float gr, float& m, float& v, const AdamHyper& h, float f) {
    const float g = gr * f + h.wd * p;
    m = h.b1 * m + h.omb1 * g;
    v = h.b2 * v + h.omb2 * g * g;
    const float mh = m / h.bc1;
    const float vh = v / h.bc2;
    p = p - h.lr * mh / (__builtin_sqrtf(vh) + h.eps);
}

// AMAX: also fold max |p| of the updated parameters into absmax[idx] (the
// binary32 bit patterns of non-negative values order like unsigned integers,
// so a global unsigned atomic max gives the exact maximum in any order).
template <bool AMAX>
__global__ __launch_bounds__(kOThreads) void adam_kernel(const AdamList L, const AdamHyper h,
                                                         const float* __restrict__ norm,
                                                         uint32_t* __restrict__ absmax) {
    uint32_t am = 0;
    float f = 1.0f;
    if (norm) {
        const float nv = norm[0];
        if (nv > h.max_norm) f = h.max_norm / nv;
    }
    const int b = blockIdx.x;
    const int t = owner(L.first, L.count, b);
    float* __restrict__ p = L.p[t];
    const float* __restrict__ g = L.g[t];
    float* __restrict__ m = L.m[t];
    float* __restrict__ v = L.v[t];
    const int64_t n = L.n[t];
    const int64_t base = (int64_t)(b - L.first[t]) * kChunk;
    if (base + kChunk <= n) {
        f32x4* pv = reinterpret_cast<f32x4*>(p + base);
        const f32x4* gv = reinterpret_cast<const f32x4*>(g + base);
        f32x4* mv = reinterpret_cast<f32x4*>(m + base);
        f32x4* vv = reinterpret_cast<f32x4*>(v + base);
        // two halves of kVec/2 float4 each: 16 loads in flight per half
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            f32x4 rp[kVec / 2], rg[kVec / 2], rm[kVec / 2], rv[kVec / 2];
#pragma unroll
            for (int k = 0; k < kVec / 2; ++k) {
                const int i = (half * (kVec / 2) + k) * kOThreads + threadIdx.x;
                rg[k] = __builtin_nontemporal_load(gv + i);
                rp[k] = __builtin_nontemporal_load(pv + i);
                rm[k] = __builtin_nontemporal_load(mv + i);
                rv[k] = __builtin_nontemporal_load(vv + i);
            }
#pragma unroll
            for (int k = 0; k < kVec / 2; ++k) {
                const int i = (half * (kVec / 2) + k) * kOThreads + threadIdx.x;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float pp = rp[k][e], mm = rm[k][e], ve = rv[k][e];
                    adam1(pp, rg[k][e], mm, ve, h, f);
                    rp[k][e] = pp;
                    rm[k][e] = mm;
                    rv[k][e] = ve;
                    if (AMAX) am = fold_f32(am, __float_as_uint(pp));
                }
                __builtin_nontemporal_store(rp[k], pv + i);
                __builtin_nontemporal_store(rm[k], mv + i);
                __builtin_nontemporal_store(rv[k], vv + i);
            }
        }
    } else {
        for (int64_t i = base + threadIdx.x; i < n; i += kOThreads) {
            float pp = p[i], mm = m[i], vv = v[i];
            adam1(pp, g[i], mm, vv, h, f);
            p[i] = pp;
            m[i] = mm;
            v[i] = vv;
            if (AMAX) am = fold_f32(am, __float_as_uint(pp));
        }
    }
    if (AMAX) {
        __shared__ uint32_t red[kOThreads / 64];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) am = max(am, (uint32_t)__shfl_xor((int)am, off, 64));
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = am;
        __syncthreads();
        if (threadIdx.x == 0) {
#pragma unroll
            for (int w = 1; w < kOThreads / 64; ++w) am = max(am, red[w]);
            atomicMax(absmax + L.idx[t], am);
        }
    }
}

static int64_t chunks(int64_t n) { return (n + kChunk - 1) / kChunk; }
static int64_t norm_chunks(int64_t n) { return (n + kNormChunk - 1) / kNormChunk; }

// Blocks of a whole list, or -1 when a launch would exceed the grid limit.
static int64_t total_blocks(const int64_t* sizes, int count) {
    int64_t b = 0;
    for (int i = 0; i < count; ++i) b += chunks(sizes[i]);
    return b;
}

// Shared argument checks of a tensor list: non-null pointers, sizes >= 0,
// 16-byte aligned pointers (the float4 path).
static int check_list(const char* fn, const void* const* ptrs, const int64_t* sizes, int count, const char* what) {
    for (int i = 0; i < count; ++i) {
        DF_CHECK(sizes[i] >= 0, DF_ERR_INVALID, "%s: %s size[%d] = %lld is negative", fn, what, i,
                 (long long)sizes[i]);
        if (sizes[i] == 0) continue;
        DF_CHECK(ptrs[i] != nullptr, DF_ERR_INVALID, "%s: %s[%d] is NULL", fn, what, i);
        DF_CHECK(aligned16(ptrs[i]), DF_ERR_ALIGN, "%s: %s[%d] is not 16-byte aligned", fn, what, i);
    }
    return DF_OK;
}

// Launches sumsq_kernel over the list in groups of kNormList tensors; the
// partials of all groups land back to back in `partial`.
static int launch_sumsq(const float* const* grads, const int64_t* sizes, int count, double* partial,
                 hipStream_t st, int* nparts) {
    int parts = 0;
    for (int i0 = 0; i0 < count;) {
        NormList L{};
        int blocks = 0;
        int c = 0;
        for (; i0 < count && c < kNormList; ++i0) {
            if (sizes[i0] == 0) continue;
            L.ptr[c] = const_cast<float*>(grads[i0]);
            L.n[c] = sizes[i0];
            L.first[c] = blocks;
            blocks += (int)norm_chunks(sizes[i0]);
            ++c;
        }
        if (c == 0) break;
        L.first[c] = blocks;
        L.count = c;
        sumsq_kernel<<<blocks, kOThreads, 0, st>>>(L, partial, parts);
        parts += blocks;
    }
    *nparts = parts;
    return launch_status("sumsq_kernel");
}

}  // namespace dfk

using namespace dfk;

extern "C" size_t df_grad_norm_workspace_bytes(int count, const int64_t* sizes) {
    if (count < 0 || (count > 0 && !sizes)) return 0;
    int64_t b = 0;
    for (int i = 0; i < count; ++i) b += sizes[i] > 0 ? norm_chunks(sizes[i]) : 0;
    return (size_t)(b > 0 ? b : 1) * sizeof(double);
}

static int grad_norm_impl(const char* fn, const float* const* grads, const int64_t* sizes, int count,
                          float* norm_dev, void* ws, size_t ws_bytes, void* stream) {
    DF_CHECK(count >= 0, DF_ERR_INVALID, "%s: count = %d is negative", fn, count);
    DF_CHECK(count == 0 || (grads && sizes), DF_ERR_INVALID, "%s: grads or sizes is NULL", fn);
    DF_CHECK(norm_dev && ws, DF_ERR_INVALID, "%s: norm_dev or ws is NULL", fn);
    DF_CHECK(aligned4(norm_dev), DF_ERR_ALIGN, "%s: norm_dev is not 4-byte aligned", fn);
    DF_CHECK(((uintptr_t)ws & 7u) == 0, DF_ERR_ALIGN, "%s: ws is not 8-byte aligned", fn);
    if (int rc = check_list(fn, reinterpret_cast<const void* const*>(grads), sizes, count, "grads")) return rc;
    const size_t need = df_grad_norm_workspace_bytes(count, sizes);
    DF_CHECK(ws_bytes >= need, DF_ERR_WORKSPACE, "%s: workspace %zu B < %zu B", fn, ws_bytes, need);
    DF_CHECK(total_blocks(sizes, count) < (1ll << 31), DF_ERR_INVALID, "%s: %lld blocks exceed the grid limit", fn,
             (long long)total_blocks(sizes, count));
    hipStream_t st = as_stream(stream);
    double* partial = static_cast<double*>(ws);
    int nparts = 0;
    if (int rc = launch_sumsq(grads, sizes, count, partial, st, &nparts)) return rc;
    // nparts == 0 (no elements): the finalize pass writes norm 0
    norm_finalize_kernel<<<1, kOThreads, 0, st>>>(partial, nparts, norm_dev);
    return launch_status("norm_finalize_kernel");
}

extern "C" int df_grad_norm_f32(const float* const* grads, const int64_t* sizes, int count, float* norm_dev,
                                void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    return grad_norm_impl("df_grad_norm_f32", grads, sizes, count, norm_dev, ws, ws_bytes, stream);
}

extern "C" int df_clip_grad_norm_f32(float* const* grads, const int64_t* sizes, int count, float max_norm,
                                     float* norm_dev, void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    const char* fn = "df_clip_grad_norm_f32";
    if (int rc = grad_norm_impl(fn, const_cast<const float* const*>(grads), sizes, count, norm_dev, ws, ws_bytes,
                                stream))
        return rc;
    hipStream_t st = as_stream(stream);
    for (int i0 = 0; i0 < count;) {
        NormList L{};
        int blocks = 0, c = 0;
        for (; i0 < count && c < kNormList; ++i0) {
            if (sizes[i0] == 0) continue;
            L.ptr[c] = grads[i0];
            L.n[c] = sizes[i0];
            L.first[c] = blocks;
            blocks += (int)chunks(sizes[i0]);
            ++c;
        }
        if (c == 0) break;
        L.first[c] = blocks;
        L.count = c;
        clip_kernel<<<blocks, kOThreads, 0, st>>>(L, norm_dev, max_norm);
    }
    return launch_status("clip_kernel");
}

// 1 - beta^t in binary32: beta^t correctly rounded to binary32 (through a
// binary64 pow), then the binary32 subtraction the reference writes
// (adam_optimizer.cu:28-29).
static float bias_correction(float beta, int t) {
    return 1.0f - (float)pow((double)beta, (double)t);
}

static int adam_impl(const char* fn, float* const* params, const float* const* grads, float* const* m,
                     float* const* v, const int64_t* sizes, int count, float lr, float beta1, float beta2, float eps,
                     float weight_decay, int timestep, const float* clip_norm_dev, float max_norm, float* absmax_dev,
                     void* stream) {
    clear_error();
    DF_CHECK(count >= 0, DF_ERR_INVALID, "%s: count = %d is negative", fn, count);
    DF_CHECK(count == 0 || (params && grads && m && v && sizes), DF_ERR_INVALID,
             "%s: a pointer array is NULL", fn);
    DF_CHECK(timestep >= 1, DF_ERR_INVALID, "%s: timestep = %d (the first step is 1)", fn, timestep);
    DF_CHECK(!clip_norm_dev || aligned4(clip_norm_dev), DF_ERR_ALIGN, "%s: clip_norm_dev misaligned", fn);
    DF_CHECK(aligned4(absmax_dev), DF_ERR_ALIGN, "%s: absmax_dev misaligned", fn);
    if (int rc = check_list(fn, reinterpret_cast<const void* const*>(params), sizes, count, "params")) return rc;
    if (int rc = check_list(fn, reinterpret_cast<const void* const*>(grads), sizes, count, "grads")) return rc;
    if (int rc = check_list(fn, reinterpret_cast<const void* const*>(m), sizes, count, "m")) return rc;
    if (int rc = check_list(fn, reinterpret_cast<const void* const*>(v), sizes, count, "v")) return rc;
    DF_CHECK(total_blocks(sizes, count) < (1ll << 31), DF_ERR_INVALID, "%s: too many elements", fn);
    AdamHyper h;
    h.lr = lr;
    h.b1 = beta1;
    h.b2 = beta2;
    h.omb1 = 1.0f - beta1;
    h.omb2 = 1.0f - beta2;
    h.eps = eps;
    h.wd = weight_decay;
    h.bc1 = bias_correction(beta1, timestep);
    h.bc2 = bias_correction(beta2, timestep);
    h.max_norm = max_norm;
    hipStream_t st = as_stream(stream);
    uint32_t* am = reinterpret_cast<uint32_t*>(absmax_dev);
    if (am && count > 0) {
        const uint32_t zero = 0;
        if (int rc = df_fill(am, count, 4, &zero, stream)) return rc;  // empty tensors stay at 0
    }
    for (int i0 = 0; i0 < count;) {
        AdamList L{};
        int blocks = 0, c = 0;
        for (; i0 < count && c < kAdamList; ++i0) {
            if (sizes[i0] == 0) continue;
            L.p[c] = params[i0];
            L.g[c] = grads[i0];
            L.m[c] = m[i0];
            L.v[c] = v[i0];
            L.n[c] = sizes[i0];
            L.first[c] = blocks;
            L.idx[c] = i0;
            blocks += (int)chunks(sizes[i0]);
            ++c;
        }
        if (c == 0) break;
        L.first[c] = blocks;
        L.count = c;
        if (am) adam_kernel<true><<<blocks, kOThreads, 0, st>>>(L, h, clip_norm_dev, am);
        else adam_kernel<false><<<blocks, kOThreads, 0, st>>>(L, h, clip_norm_dev, nullptr);
    }
    return launch_status("adam_kernel");
}

extern "C" int df_adam_update_f32(float* const* params, const float* const* grads, float* const* m,
                                  float* const* v, const int64_t* sizes, int count, float lr, float beta1,
                                  float beta2, float eps, float weight_decay, int timestep,
                                  const float* clip_norm_dev, float max_norm, void* stream) {
    return adam_impl("df_adam_update_f32", params, grads, m, v, sizes, count, lr, beta1, beta2, eps, weight_decay,
                     timestep, clip_norm_dev, max_norm, nullptr, stream);
}

extern "C" int df_adam_update_absmax_f32(float* const* params, const float* const* grads, float* const* m,
                                         float* const* v, const int64_t* sizes, int count, float lr, float beta1,
                                         float beta2, float eps, float weight_decay, int timestep,
                                         const float* clip_norm_dev, float max_norm, float* absmax_dev,
                                         void* stream) {
    DF_CHECK(absmax_dev || count == 0, DF_ERR_INVALID, "df_adam_update_absmax_f32: absmax_dev is NULL");
    return adam_impl("df_adam_update_absmax_f32", params, grads, m, v, sizes, count, lr, beta1, beta2, eps,
                     weight_decay, timestep, clip_norm_dev, max_norm, absmax_dev, stream);
}
