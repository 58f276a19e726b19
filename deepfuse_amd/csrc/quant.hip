// quant.hip -- absmax, scale, quantize and dequantize kernels (gfx950).
//
// All four are HBM-bandwidth kernels.  Layout: flat, contiguous tensors.
// Each thread moves 16 bytes per global load (dwordx4) on the wide side of
// the conversion, a wave covers 1 KiB contiguous per instruction, and the
// grid is a fixed multiple of the CU count with a grid-stride loop so every
// CU keeps several loads in flight.
//
// Reference: the reference has no quantizer (README.md:16 claim only; fp8 is
// a type at dnn/core/tensor.cu:489-498).  Semantics: include/df_capi.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "df_common.hpp"

namespace dfk {

constexpr int kThreads = 256;
constexpr int kMaxReduceBlocks = 2048;  // partials in the absmax workspace
// absmax blocks of df_quantize_2d_jit: every tile block folds their
// partials, so fewer than kMaxReduceBlocks (512: 2 KiB per tile block, and
// still enough blocks for the absmax pass to stream at full rate)
constexpr int kJitParts = 512;

// ------------------------------------------------------------------ absmax --
// (fold_f32 and fold_bf16x2, the binary32 and bf16-pair folds, are in df_common.hpp)

__device__ __forceinline__ uint32_t block_max_u32(uint32_t m) {
    __shared__ uint32_t red[kThreads / 64];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off, 64));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 1; w < kThreads / 64; ++w) m = max(m, red[w]);
    }
    return m;  // valid in thread 0
}

// Streaming layout shared by the flat kernels: the vector index space (16
// bytes of input per vector) is cut into chunks of kThreads * kU vectors;
// block b takes chunks b, b + G, ... and each thread issues kU 16-byte
// loads, kThreads apart, before using any of them (a wave instruction
// covers 1 KiB contiguous).  Only the last, partial chunk takes the
// element-guarded loop.
constexpr int kU = 8;
constexpr int64_t kChunkVec = (int64_t)kThreads * kU;
// Loads per thread and chunk of the flat conversions (the absmax reads keep
// kU).  The fp32 conversions run best at 2048 elements per 256-thread block
// (config 2, one MI355X, alternating runs on one box): fp8 -> fp32 5.85 ->
// 6.21-6.37 TB/s going from 8 to 2 vectors per thread, fp8 -> bf16
// 5.97-6.01 -> 6.29-6.36 from 8 to 1, fp32 -> fp8 6.08-6.11 -> 6.28-6.36
// from 8 to 2.  bf16 -> fp8 issues 4: 6.17-6.22 -> 6.24-6.30 TB/s from 8
// (at 2, 5.83-6.08).
constexpr int kUQuantF32 = 2, kUQuantBf16 = 4, kUDeqF32 = 2, kUDeqBf16 = 1;

// Stage 1 bodies: the block's maximum over its chunks (block bi of nb
// blocks walking the chunks with a stride of nb).  |x| bit patterns, NaN
// and infinities skipped (fold_*).
__device__ __forceinline__ uint32_t absmax_f32_block(const float* __restrict__ x, int64_t n, int bi, int nb) {
    uint32_t m = 0;
    const int64_t nvec = n >> 2;
    const u32x4* xv = reinterpret_cast<const u32x4*>(x);
    for (int64_t base = (int64_t)bi * kChunkVec; base < nvec; base += (int64_t)nb * kChunkVec) {
        if (base + kChunkVec <= nvec) {
            u32x4 v[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) v[u] = __builtin_nontemporal_load(xv + base + u * kThreads + threadIdx.x);
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                m = fold_f32(m, v[u].x); m = fold_f32(m, v[u].y); m = fold_f32(m, v[u].z); m = fold_f32(m, v[u].w);
            }
        } else {
            for (int64_t i = base + threadIdx.x; i < nvec; i += kThreads) {
                const u32x4 v = xv[i];
                m = fold_f32(m, v.x); m = fold_f32(m, v.y); m = fold_f32(m, v.z); m = fold_f32(m, v.w);
            }
        }
    }
    if (bi == 0 && threadIdx.x < (n & 3))
        m = fold_f32(m, __float_as_uint(x[(nvec << 2) + threadIdx.x]));
    return block_max_u32(m);
}

// bf16: 16-byte loads hold 8 values.
__device__ __forceinline__ uint32_t absmax_bf16_block(const uint16_t* __restrict__ x, int64_t n, int bi, int nb) {
    uint32_t m = 0;
    const int64_t nvec = n >> 3;
    const u32x4* xv = reinterpret_cast<const u32x4*>(x);
    for (int64_t base = (int64_t)bi * kChunkVec; base < nvec; base += (int64_t)nb * kChunkVec) {
        if (base + kChunkVec <= nvec) {
            u32x4 v[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) v[u] = __builtin_nontemporal_load(xv + base + u * kThreads + threadIdx.x);
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                m = fold_bf16x2(m, v[u].x); m = fold_bf16x2(m, v[u].y);
                m = fold_bf16x2(m, v[u].z); m = fold_bf16x2(m, v[u].w);
            }
        } else {
            for (int64_t i = base + threadIdx.x; i < nvec; i += kThreads) {
                const u32x4 v = xv[i];
                m = fold_bf16x2(m, v.x); m = fold_bf16x2(m, v.y); m = fold_bf16x2(m, v.z); m = fold_bf16x2(m, v.w);
            }
        }
    }
    if (bi == 0 && threadIdx.x < (n & 7))
        m = fold_f32(m, (uint32_t)x[(nvec << 3) + threadIdx.x] << 16);
    return block_max_u32(m);
}

// binary16: 16-byte loads hold 8 values, each widened exactly.
__device__ __forceinline__ uint32_t fold_f16x2(uint32_t m, uint32_t w) {
    m = fold_f32(m, __float_as_uint(f16_to_f32(w & 0xFFFFu)));
    return fold_f32(m, __float_as_uint(f16_to_f32(w >> 16)));
}
__device__ __forceinline__ uint32_t absmax_f16_block(const uint16_t* __restrict__ x, int64_t n, int bi, int nb) {
    uint32_t m = 0;
    const int64_t nvec = n >> 3;
    const u32x4* xv = reinterpret_cast<const u32x4*>(x);
    for (int64_t base = (int64_t)bi * kChunkVec; base < nvec; base += (int64_t)nb * kChunkVec) {
        if (base + kChunkVec <= nvec) {
            u32x4 v[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) v[u] = __builtin_nontemporal_load(xv + base + u * kThreads + threadIdx.x);
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                m = fold_f16x2(m, v[u].x); m = fold_f16x2(m, v[u].y);
                m = fold_f16x2(m, v[u].z); m = fold_f16x2(m, v[u].w);
            }
        } else {
            for (int64_t i = base + threadIdx.x; i < nvec; i += kThreads) {
                const u32x4 v = xv[i];
                m = fold_f16x2(m, v.x); m = fold_f16x2(m, v.y); m = fold_f16x2(m, v.z); m = fold_f16x2(m, v.w);
            }
        }
    }
    if (bi == 0 && threadIdx.x < (n & 7))
        m = fold_f32(m, __float_as_uint(f16_to_f32(x[(nvec << 3) + threadIdx.x])));
    return block_max_u32(m);
}

// Stage 1: one partial maximum per block.
__global__ __launch_bounds__(kThreads) void absmax_f32_stage1(const float* __restrict__ x, int64_t n,
                                                               uint32_t* __restrict__ partial) {
    const uint32_t m = absmax_f32_block(x, n, blockIdx.x, gridDim.x);
    if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

__global__ __launch_bounds__(kThreads) void absmax_bf16_stage1(const uint16_t* __restrict__ x, int64_t n,
                                                                uint32_t* __restrict__ partial) {
    const uint32_t m = absmax_bf16_block(x, n, blockIdx.x, gridDim.x);
    if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

__global__ __launch_bounds__(kThreads) void absmax_f16_stage1(const uint16_t* __restrict__ x, int64_t n,
                                                               uint32_t* __restrict__ partial) {
    const uint32_t m = absmax_f16_block(x, n, blockIdx.x, gridDim.x);
    if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// scale rule D1/D2: s = absmax / fmax (IEEE division); absmax == 0 or a
// scale that is not a positive finite number gives 1.
__device__ __forceinline__ float scale_from_absmax(float am, int fmt) {
    const float fmax = fmt == E4M3 ? Fp8<E4M3>::fmax : Fp8<E5M2>::fmax;
    if (!(am > 0.0f) || !(am <= 3.4028234663852886e38f)) return 1.0f;
    const float s = am / fmax;
    return (s > 0.0f && s <= 3.4028234663852886e38f) ? s : 1.0f;
}

// Stage 2: one block folds the partials, writes absmax and (optionally) scale.
// This thread's max over partial[threadIdx.x + k * kThreads]: eight
// independent loads in flight per iteration (one iteration for 2048
// partials), not one load-then-max chain per partial.
__device__ __forceinline__ uint32_t fold_parts(const uint32_t* __restrict__ partial, int nparts) {
    uint32_t m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = threadIdx.x;
    for (; i + 7 * kThreads < nparts; i += 8 * kThreads) {
#pragma unroll
        for (int u = 0; u < 8; ++u) m[u] = max(m[u], partial[i + u * kThreads]);
    }
    for (; i < nparts; i += kThreads) m[0] = max(m[0], partial[i]);
    return max(max(max(m[0], m[1]), max(m[2], m[3])), max(max(m[4], m[5]), max(m[6], m[7])));
}

__global__ __launch_bounds__(kThreads) void absmax_stage2(const uint32_t* __restrict__ partial,
                                                           int nparts, int fmt,
                                                           float* __restrict__ absmax_out,
                                                           float* __restrict__ scale_out) {
    uint32_t m = block_max_u32(fold_parts(partial, nparts));
    if (threadIdx.x == 0) {
        const float am = __uint_as_float(m);
        if (absmax_out) absmax_out[0] = am;
        if (scale_out) scale_out[0] = scale_from_absmax(am, fmt);
    }
}

void launch_absmax_fold(const uint32_t* partial, int nparts, int fmt, float* absmax_out, float* scale_out,
                        hipStream_t st) {
    absmax_stage2<<<1, kThreads, 0, st>>>(partial, nparts, fmt, absmax_out, scale_out);
}

// Stage 2 folded into the pass that uses the scale (no one-block launch
// between them): every block of that pass folds the stage-1 partials itself,
// gets the same maximum, and forms the scale by rule D1/D2; the writer block
// also stores absmax and scale for the caller.  The barrier at the end hands
// the scale to every thread and keeps block_max_u32's LDS free for reuse.
struct JitScale {
    const uint32_t* parts = nullptr;
    int nparts = 0;
    float* absmax_out = nullptr;
    float* scale_out = nullptr;
};

__device__ __forceinline__ float jit_block_scale(const uint32_t* __restrict__ parts, int nparts, int fmt,
                                                 float* __restrict__ absmax_out, float* __restrict__ scale_out,
                                                 bool writer) {
    __shared__ float s_scale;
    const uint32_t m = block_max_u32(fold_parts(parts, nparts));
    if (threadIdx.x == 0) {
        const float am = __uint_as_float(m), sc = scale_from_absmax(am, fmt);
        s_scale = sc;
        if (writer) {
            if (absmax_out) absmax_out[0] = am;
            if (scale_out) scale_out[0] = sc;
        }
    }
    __syncthreads();
    return s_scale;
}

__global__ void scale_kernel(const float* __restrict__ absmax, int fmt, float* __restrict__ scale) {
    if (threadIdx.x == 0) scale[0] = scale_from_absmax(absmax[0], fmt);
}

// ---------------------------------------------------------------- quantize --
// x / s (correctly rounded: qdiv, contract D1), then the fp8 encoder
// (encode2_hw: hardware round-to-nearest-even after saturation, NaN kept).

// plain or non-temporal (NT) accesses.  The flat kernels store
// non-temporal (NTS) when their output starts on a 128-byte boundary: every
// wave store then covers whole cache lines.  A misaligned output takes plain
// stores, so no line is assembled from several non-temporal partial writes
// of neighbouring blocks.
template <bool NT, typename T> __device__ __forceinline__ T ld_nt(const T* p) {
    if (NT) return __builtin_nontemporal_load(p);
    return *p;
}
template <bool NT, typename T> __device__ __forceinline__ void st_nt(T* p, const T v) {
    if (NT)
        __builtin_nontemporal_store(v, p);
    else
        *p = v;
}

// fp32 -> fp8: a 16-byte load of 4 values -> a 4-byte store of 4 codes.
template <int FMT, bool FAST, bool NTS>
__device__ __forceinline__ void quantize_f32_body(const float* __restrict__ x, int64_t n, const QDiv& d,
                                                  uint8_t* __restrict__ q) {
    constexpr int U = kUQuantF32;
    constexpr int64_t CH = (int64_t)kThreads * U;
    const int64_t nvec = n >> 2;
    const f32x4* xv = reinterpret_cast<const f32x4*>(x);
    uint32_t* qv = reinterpret_cast<uint32_t*>(q);
    for (int64_t base = (int64_t)blockIdx.x * CH; base < nvec; base += (int64_t)gridDim.x * CH) {
        if (base + CH <= nvec) {
            f32x4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(xv + base + u * kThreads + threadIdx.x);
            const float* t = reinterpret_cast<const float*>(v);
            if (FAST && !wave_any_nan<4 * U>(t)) {
#pragma unroll
                for (int u = 0; u < U; ++u)
                    st_nt<NTS>(qv + base + u * kThreads + threadIdx.x,
                               quant4_nonan<FMT>(v[u].x, v[u].y, v[u].z, v[u].w, d));
            } else {
#pragma unroll
                for (int u = 0; u < U; ++u)
                    st_nt<NTS>(qv + base + u * kThreads + threadIdx.x,
                               quant4_t<FMT, FAST>(v[u].x, v[u].y, v[u].z, v[u].w, d));
            }
        } else {
            for (int64_t i = base + threadIdx.x; i < nvec; i += kThreads) {
                const f32x4 v = xv[i];
                qv[i] = quant4_t<FMT, FAST>(v.x, v.y, v.z, v.w, d);
            }
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        const int64_t j = (nvec << 2) + threadIdx.x;
        q[j] = (uint8_t)encode2_hw<FMT>(qdiv_t<FAST>(x[j], d), 0.0f);
    }
}

template <int FMT, bool NTS>
__global__ __launch_bounds__(kThreads) void quantize_f32_kernel(const float* __restrict__ x,
                                                                 int64_t n,
                                                                 const float* __restrict__ scale,
                                                                 uint8_t* __restrict__ q) {
    const QDiv d = make_qdiv(scale[0]);
    if (d.fast)
        quantize_f32_body<FMT, true, NTS>(x, n, d, q);
    else
        quantize_f32_body<FMT, false, NTS>(x, n, d, q);
}

// bf16 -> fp8: one 16-byte load (8 values) -> one 8-byte store.
template <int FMT, bool FAST>
__device__ __forceinline__ uint32_t quant_bf16x4(uint32_t w0, uint32_t w1, const QDiv& d) {
    return quant4_t<FMT, FAST>(bf16_to_f32(w0 & 0xFFFFu), bf16_to_f32(w0 >> 16), bf16_to_f32(w1 & 0xFFFFu),
                               bf16_to_f32(w1 >> 16), d);
}

// eight bf16 values of one 16-byte load -> eight codes
template <int FMT, bool FAST>
__device__ __forceinline__ u32x2 quant_bf16x8(const u32x4 w, const QDiv& d) {
    const float t[8] = {bf16_to_f32(w.x & 0xFFFFu), bf16_to_f32(w.x >> 16), bf16_to_f32(w.y & 0xFFFFu),
                        bf16_to_f32(w.y >> 16),     bf16_to_f32(w.z & 0xFFFFu), bf16_to_f32(w.z >> 16),
                        bf16_to_f32(w.w & 0xFFFFu), bf16_to_f32(w.w >> 16)};
    u32x2 o;
    if (FAST && !wave_any_nan<8>(t)) {
        o.x = quant4_nonan<FMT>(t[0], t[1], t[2], t[3], d);
        o.y = quant4_nonan<FMT>(t[4], t[5], t[6], t[7], d);
    } else {
        o.x = quant4_t<FMT, FAST>(t[0], t[1], t[2], t[3], d);
        o.y = quant4_t<FMT, FAST>(t[4], t[5], t[6], t[7], d);
    }
    return o;
}

template <int FMT, bool FAST, bool NTS>
__device__ __forceinline__ void quantize_bf16_body(const uint16_t* __restrict__ x, int64_t n, const QDiv& d,
                                                   uint8_t* __restrict__ q) {
    constexpr int U = kUQuantBf16;
    constexpr int64_t CH = (int64_t)kThreads * U;
    const int64_t nvec = n >> 3;
    const u32x4* xv = reinterpret_cast<const u32x4*>(x);
    u32x2* qv = reinterpret_cast<u32x2*>(q);
    for (int64_t base = (int64_t)blockIdx.x * CH; base < nvec; base += (int64_t)gridDim.x * CH) {
        if (base + CH <= nvec) {
            u32x4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(xv + base + u * kThreads + threadIdx.x);
#pragma unroll
            for (int u = 0; u < U; ++u)
                st_nt<NTS>(qv + base + u * kThreads + threadIdx.x, quant_bf16x8<FMT, FAST>(v[u], d));
        } else {
            for (int64_t i = base + threadIdx.x; i < nvec; i += kThreads) {
                const u32x4 v = xv[i];
                u32x2 o;
                o.x = quant_bf16x4<FMT, FAST>(v.x, v.y, d);
                o.y = quant_bf16x4<FMT, FAST>(v.z, v.w, d);
                qv[i] = o;
            }
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 7)) {
        const int64_t j = (nvec << 3) + threadIdx.x;
        q[j] = (uint8_t)encode2_hw<FMT>(qdiv_t<FAST>(bf16_to_f32(x[j]), d), 0.0f);
    }
}

template <int FMT, bool NTS>
__global__ __launch_bounds__(kThreads) void quantize_bf16_kernel(const uint16_t* __restrict__ x,
                                                                  int64_t n,
                                                                  const float* __restrict__ scale,
                                                                  uint8_t* __restrict__ q) {
    const QDiv d = make_qdiv(scale[0]);
    if (d.fast)
        quantize_bf16_body<FMT, true, NTS>(x, n, d, q);
    else
        quantize_bf16_body<FMT, false, NTS>(x, n, d, q);
}

// -------------------------------------------------------------- dequantize --
// bf16 output: codes decode with the hardware conversion (v_cvt_pk_f32_fp8 /
// _bf8: two OCP codes of a dword half to binary32, exact; infinities stay
// infinite), then the multiply by s, the code's sign copied onto the result
// and the rounding by v_cvt_pk_bf16_f32 (nearest even; a quiet NaN keeps its
// sign).  The sign copy changes nothing but NaN codes, which the conversion
// returns as the negative quiet NaN 0xFFC00000 whatever their sign (D5 keeps
// the code's sign).  About four operations per element where the bit-level
// decode and rounding in software (decode_fp8, f32_to_bf16_rne) took about
// twelve: e5m2 -> bf16 went from 5.37-5.65 to 6.02 TB/s, e4m3 -> bf16 from
// 5.77-5.82 to 6.00 (config 2, one box).  fp32 output keeps the software
// decode: with the hardware one it ran 12% slower (5.15-5.22 against
// 5.86-5.91 TB/s on the same box).  The all-codes tests pin both forms.
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

template <int FMT, bool HI>
__device__ __forceinline__ v2f decode2_hw(uint32_t w) {
    if constexpr (FMT == E4M3)
        return __builtin_amdgcn_cvt_pk_f32_fp8(w, HI);
    else
        return __builtin_amdgcn_cvt_pk_f32_bf8(w, HI);
}
// v with the sign of bit 31 of w (the sign bit of the code shifted there)
__device__ __forceinline__ float with_sign_of(float v, uint32_t w) {
    return __builtin_copysignf(v, __uint_as_float(w));
}
__device__ __forceinline__ uint32_t pack_bf16_hw(float a, float b) {
    const v2f f = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, v2bf));
}

// fp8 -> fp32: a 4-byte load (4 codes) -> a 16-byte store; the chunks count
// output vectors.
template <int FMT, bool NTS>
__global__ __launch_bounds__(kThreads) void dequantize_f32_kernel(const uint8_t* __restrict__ q,
                                                                   int64_t n,
                                                                   const float* __restrict__ scale,
                                                                   float* __restrict__ out) {
    const float s = scale[0];
    const int64_t nvec = n >> 2;
    const uint32_t* qv = reinterpret_cast<const uint32_t*>(q);
    f32x4* ov = reinterpret_cast<f32x4*>(out);
    auto deq4 = [&](uint32_t w) {
        f32x4 o;
        o.x = dequant_fp8<FMT>(w & 0xFFu, s);
        o.y = dequant_fp8<FMT>((w >> 8) & 0xFFu, s);
        o.z = dequant_fp8<FMT>((w >> 16) & 0xFFu, s);
        o.w = dequant_fp8<FMT>(w >> 24, s);
        return o;
    };
    constexpr int U = kUDeqF32;
    constexpr int64_t CH = (int64_t)kThreads * U;
    for (int64_t base = (int64_t)blockIdx.x * CH; base < nvec; base += (int64_t)gridDim.x * CH) {
        if (base + CH <= nvec) {
            uint32_t w[U];
#pragma unroll
            for (int u = 0; u < U; ++u) w[u] = __builtin_nontemporal_load(qv + base + u * kThreads + threadIdx.x);
#pragma unroll
            for (int u = 0; u < U; ++u) st_nt<NTS>(ov + base + u * kThreads + threadIdx.x, deq4(w[u]));
        } else {
            for (int64_t i = base + threadIdx.x; i < nvec; i += kThreads) ov[i] = deq4(qv[i]);
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        const int64_t j = (nvec << 2) + threadIdx.x;
        out[j] = dequant_fp8<FMT>(q[j], s);
    }
}

// fp8 -> bf16: one 8-byte load (8 codes) -> one 16-byte store.
template <int FMT, bool HI>
__device__ __forceinline__ uint32_t deq_bf16x2(uint32_t w, float s) {
    const v2f v = decode2_hw<FMT, HI>(w);
    return pack_bf16_hw(with_sign_of(v.x * s, w << (HI ? 8 : 24)), with_sign_of(v.y * s, w << (HI ? 0 : 16)));
}

template <int FMT, bool NTS>
__global__ __launch_bounds__(kThreads) void dequantize_bf16_kernel(const uint8_t* __restrict__ q,
                                                                    int64_t n,
                                                                    const float* __restrict__ scale,
                                                                    uint16_t* __restrict__ out) {
    const float s = scale[0];
    const int64_t nvec = n >> 3;
    const u32x2* qv = reinterpret_cast<const u32x2*>(q);
    u32x4* ov = reinterpret_cast<u32x4*>(out);
    auto deq8 = [&](u32x2 w) {
        return u32x4{deq_bf16x2<FMT, false>(w.x, s), deq_bf16x2<FMT, true>(w.x, s), deq_bf16x2<FMT, false>(w.y, s),
                     deq_bf16x2<FMT, true>(w.y, s)};
    };
    constexpr int U = kUDeqBf16;
    constexpr int64_t CH = (int64_t)kThreads * U;
    for (int64_t base = (int64_t)blockIdx.x * CH; base < nvec; base += (int64_t)gridDim.x * CH) {
        if (base + CH <= nvec) {
            u32x2 w[U];
#pragma unroll
            for (int u = 0; u < U; ++u) w[u] = __builtin_nontemporal_load(qv + base + u * kThreads + threadIdx.x);
#pragma unroll
            for (int u = 0; u < U; ++u) st_nt<NTS>(ov + base + u * kThreads + threadIdx.x, deq8(w[u]));
        } else {
            for (int64_t i = base + threadIdx.x; i < nvec; i += kThreads) ov[i] = deq8(qv[i]);
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 7)) {
        const int64_t j = (nvec << 3) + threadIdx.x;
        out[j] = (uint16_t)(pack_bf16_hw(with_sign_of(decode2_hw<FMT, false>(q[j]).x * s, (uint32_t)q[j] << 24),
                                         0.0f) &
                            0xFFFFu);
    }
}

// ------------------------------------------------------- 2-D + transposed --
// One 128 x 128 tile per 256-thread block.  Thread t owns the 16-byte
// column chunk (t % TPR) of RPT consecutive rows: 16-byte loads, row-major
// codes stored straight to q, and the same codes written transposed into an
// LDS tile [column][row] that is then stored to qt as 128-byte row segments.
// Elements outside [rows) x [cols) encode as 0, so the padding of q (columns
// up to ldq) and of qt (columns up to ldqt) is written in the same pass.
// NT (default: AMAX without LN, i.e. delayed scaling, where no absmax or
// statistics pass has just read x) makes the loads of x and the stores of
// q / qt non-temporal.  On the 16384 x {1600, 4800, 6400} bf16 operands of
// GPT-2 XL that made the delayed-scaling config-4 step about 2% faster
// (2.001-2.016 ms against 2.039-2.057 ms, alternating runs on one box);
// after an absmax pass the cached re-read of x hits the Infinity Cache and
// plain accesses are faster.
// With COLSUM the block also folds the fp32 values of its tile into one
// partial sum per column (rows in fixed order), written to
// colpart[tile_row][col] for a deterministic second pass.
constexpr int kT2 = 128;
// rows of a quantize_2d_kernel tile (quantize_2d_batch_kernel keeps kT2)
constexpr int kT2R = 128;

// LDS layout of a tile's transposed codes: column col holds the 128 codes
// of its rows as sixteen 8-byte slots (slot s = rows 8s..8s+7).  Columns
// are paired into 256-byte units, and the 32 slots of a pair are permuted
// by an even XOR key taken from the column's thread group (col / E, E =
// the columns one thread loads), so
//  - the 8- or 16-byte writes of one instruction (one column per thread
//    group, the row slots of the block's row groups) spread over all 64
//    banks instead of landing 16 to a bank (a column stride that is a
//    multiple of the bank period did that), and
//  - a 16-byte chunk (slots 2j, 2j+1) stays contiguous and aligned, so the
//    read-back of 16 rows of one column is one ds_read_b128, and the 16
//    lanes reading one column pair hit distinct banks.
template <int E>
__device__ __forceinline__ int tslot(int col, int s) {
    const int key = ((col / E) & 15) << 1;
    return (col >> 1) * 256 + (((((col & 1) << 4) | s) ^ key) << 3);
}

template <typename InT> struct Ld;
template <> struct Ld<float> {
    static constexpr int E = 4;
    static __device__ __forceinline__ void widen(const u32x4 t, float* v) {
        v[0] = __uint_as_float(t.x); v[1] = __uint_as_float(t.y);
        v[2] = __uint_as_float(t.z); v[3] = __uint_as_float(t.w);
    }
    static __device__ __forceinline__ void vec(const float* p, float* v) {
        widen(*reinterpret_cast<const u32x4*>(p), v);
    }
    static __device__ __forceinline__ float one(const float* p) { return *p; }
};
template <> struct Ld<uint16_t> {
    static constexpr int E = 8;
    static __device__ __forceinline__ void widen(const u32x4 t, float* v) {
        const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = bf16_to_f32(w[i] & 0xFFFFu);
            v[2 * i + 1] = bf16_to_f32(w[i] >> 16);
        }
    }
    static __device__ __forceinline__ void vec(const uint16_t* p, float* v) {
        widen(*reinterpret_cast<const u32x4*>(p), v);
    }
    static __device__ __forceinline__ float one(const uint16_t* p) { return bf16_to_f32(*p); }
};
template <> struct Ld<f16_t> {
    static constexpr int E = 8;
    static __device__ __forceinline__ void widen(const u32x4 t, float* v) {
        const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = f16_to_f32(w[i] & 0xFFFFu);
            v[2 * i + 1] = f16_to_f32(w[i] >> 16);
        }
    }
    static __device__ __forceinline__ void vec(const f16_t* p, float* v) {
        widen(*reinterpret_cast<const u32x4*>(p), v);
    }
    static __device__ __forceinline__ float one(const f16_t* p) { return f16_to_f32(p->bits); }
};

// ---------------------------------------------------------------- LayerNorm --
// Row statistics and the per-element map of the reference's
// layer_norm_forward_kernel (dnn/layers/layer_norm_layer.cu:26-63):
//   y = (x - mean) * rstd [* gamma + beta],  mean = sum/C, var = sum((x-mean)^2)/C,
//   rstd = 1 / sqrt(var + eps)
// then rounded to the tensor's element type (the reference casts to T).
// The statistics kernel and the tile kernel evaluate y with the same
// operations on the same stored (mean, rstd), so the absmax the first
// measures is the absmax of the values the second quantizes.
struct LnArgs {
    const float2* stat = nullptr;  // (mean, rstd) per row
    const void* gamma = nullptr;   // [cols] in the input type, NULL: no affine map
    const void* beta = nullptr;
    void* y = nullptr;             // optional output [rows, ldy] in the input type
    int ldy = 0;
    bool y_vec = false;            // y and ldy allow 16-byte row stores
};

template <typename InT> __device__ __forceinline__ float round_to(float v);
template <> __device__ __forceinline__ float round_to<float>(float v) { return v; }
template <> __device__ __forceinline__ float round_to<uint16_t>(float v) { return bf16_to_f32(f32_to_bf16_rne(v)); }
template <> __device__ __forceinline__ float round_to<f16_t>(float v) { return f16_to_f32(f32_to_f16_rne(v)); }

template <typename InT> __device__ __forceinline__ void store_one(InT* p, float v);
template <> __device__ __forceinline__ void store_one<float>(float* p, float v) { *p = v; }
template <> __device__ __forceinline__ void store_one<uint16_t>(uint16_t* p, float v) {
    *p = (uint16_t)f32_to_bf16_rne(v);
}
template <> __device__ __forceinline__ void store_one<f16_t>(f16_t* p, float v) {
    p->bits = (uint16_t)f32_to_f16_rne(v);
}
// 16 bytes of values already rounded to the element type
template <typename InT> __device__ __forceinline__ void store_vec(InT* p, const float* v);
template <> __device__ __forceinline__ void store_vec<float>(float* p, const float* v) {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
}
template <> __device__ __forceinline__ void store_vec<uint16_t>(uint16_t* p, const float* v) {
    u32x4 w;
    w.x = (__float_as_uint(v[0]) >> 16) | (__float_as_uint(v[1]) & 0xFFFF0000u);
    w.y = (__float_as_uint(v[2]) >> 16) | (__float_as_uint(v[3]) & 0xFFFF0000u);
    w.z = (__float_as_uint(v[4]) >> 16) | (__float_as_uint(v[5]) & 0xFFFF0000u);
    w.w = (__float_as_uint(v[6]) >> 16) | (__float_as_uint(v[7]) & 0xFFFF0000u);
    *reinterpret_cast<u32x4*>(p) = w;
}
template <> __device__ __forceinline__ void store_vec<f16_t>(f16_t* p, const float* v) {
    u32x4 w;
    w.x = f32_to_f16_rne(v[0]) | (f32_to_f16_rne(v[1]) << 16);
    w.y = f32_to_f16_rne(v[2]) | (f32_to_f16_rne(v[3]) << 16);
    w.z = f32_to_f16_rne(v[4]) | (f32_to_f16_rne(v[5]) << 16);
    w.w = f32_to_f16_rne(v[6]) | (f32_to_f16_rne(v[7]) << 16);
    *reinterpret_cast<u32x4*>(p) = w;
}

template <typename InT>
__device__ __forceinline__ float ln_apply(float x, float mean, float rstd, bool affine, float g, float b) {
    float n = (x - mean) * rstd;
    if (affine) n = __builtin_fmaf(n, g, b);
    return round_to<InT>(n);
}


// With AMAX the block also folds |x| over finite values of its tile into one
// partial maximum (binary32 bit pattern), amaxpart[tile index], for the
// delayed-scaling history.  With LN the tile holds LayerNorm outputs: each
// loaded x becomes ln_apply(x, row stats, column gamma/beta), written to
// ln.y when given, and those values are what the codes, column sums and
// absmax see.
// The tile pass proper, instantiated for both division forms (FAST: see
// qdiv_t); the kernel below owns the LDS and picks the form once per block.
template <typename InT, int FMT, bool COLSUM, bool CODES, bool AMAX, bool LN, bool FAST, bool NT = AMAX && !LN,
          int TR = kT2>
__device__ __forceinline__ void q2d_tile(const InT* __restrict__ x, int rows, int cols, int ldx, bool vec_ok,
                                         const QDiv& d, uint8_t* __restrict__ q, int ldq, uint8_t* __restrict__ qt,
                                         int ldqt, float* __restrict__ colpart, uint32_t* __restrict__ amaxpart,
                                         const LnArgs& ln, uint8_t* tile, float (*csum)[kT2], int bx, int by,
                                         int nbx) {
    constexpr int E = Ld<InT>::E;      // elements per 16-byte load
    constexpr int TPR = kT2 / E;       // threads per tile row
    constexpr int RG = kThreads / TPR; // row groups
    constexpr int RPT = TR / RG;       // rows per thread (8 for bf16, 16 for fp32 at TR = 128)
    static_assert(RPT % 4 == 0 && RPT <= 32, "4x4 byte transposes");
    static_assert(TR == 128 && (RPT == 8 || RPT == 16), "the tslot layout holds 128-row tiles, 8 or 16 rows a thread");
    const int r0 = by * TR, c0 = bx * kT2;  // tile (bx, by) of a grid nbx tiles wide
    const int tc = (threadIdx.x % TPR) * E, rg = threadIdx.x / TPR;
    const int c = c0 + tc;
    const bool full = vec_ok && c + E <= cols;
    // Non-temporal stores only where each 128-byte row segment a block
    // writes is one whole cache line (output and its row stride 128-byte
    // aligned), so no line is assembled from several non-temporal partial
    // writes; other layouts take plain stores.
    const bool q_lines = ((reinterpret_cast<uintptr_t>(q) | (uint32_t)ldq) & 127u) == 0;
    const bool qt_lines = TR % 128 == 0 && ((reinterpret_cast<uintptr_t>(qt) | (uint32_t)ldqt) & 127u) == 0;
    uint32_t codes[RPT][E / 4];
    float cs[E];
    uint32_t am = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) cs[e] = 0.0f;
    float lg[LN ? E : 1], lb[LN ? E : 1];
    const bool affine = LN && ln.gamma != nullptr;
    if (LN) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const bool in = c + e < cols;
            lg[e] = affine && in ? Ld<InT>::one(static_cast<const InT*>(ln.gamma) + c + e) : 0.0f;
            lb[e] = affine && in ? Ld<InT>::one(static_cast<const InT*>(ln.beta) + c + e) : 0.0f;
        }
    }
    // everything after the load of one row's E values
    auto row = [&](int rr, float* v) {
        const int r = r0 + rg * RPT + rr;
        if (LN && r < rows) {
            const float2 st = ln.stat[r];
#pragma unroll
            for (int e = 0; e < E; ++e)
                v[e] = c + e < cols ? ln_apply<InT>(v[e], st.x, st.y, affine, lg[e], lb[e]) : 0.0f;
            if (ln.y) {
                InT* yr = static_cast<InT*>(ln.y) + (int64_t)r * ln.ldy + c;
                if (full && ln.y_vec) {
                    store_vec<InT>(yr, v);
                } else {
#pragma unroll
                    for (int e = 0; e < E; ++e)
                        if (c + e < cols) store_one<InT>(yr + e, v[e]);
                }
            }
        }
        if (COLSUM) {
#pragma unroll
            for (int e = 0; e < E; ++e) cs[e] += v[e];
        }
        if (AMAX) {
#pragma unroll
            for (int e = 0; e < E; ++e) am = fold_f32(am, __float_as_uint(v[e]));
        }
        if (!CODES) return;
        if (FAST && !wave_any_nan<E>(v)) {
#pragma unroll
            for (int g = 0; g < E / 4; ++g)
                codes[rr][g] = quant4_nonan<FMT>(v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3], d);
        } else {
#pragma unroll
            for (int g = 0; g < E / 4; ++g)
                codes[rr][g] = quant4_t<FMT, FAST>(v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3], d);
        }
        if (q && r < rows && c < ldq) {
            uint8_t* const dst = q + (int64_t)r * ldq + c;
            if (NT && q_lines) {
                if (E == 8)
                    st_nt<true>(reinterpret_cast<u32x2*>(dst), u32x2{codes[rr][0], codes[rr][E / 4 - 1]});
                else
                    st_nt<true>(reinterpret_cast<uint32_t*>(dst), codes[rr][0]);
            } else {
                if (E == 8)
                    *reinterpret_cast<u32x2*>(dst) = u32x2{codes[rr][0], codes[rr][E / 4 - 1]};
                else
                    *reinterpret_cast<uint32_t*>(dst) = codes[rr][0];
            }
        }
    };
    if (full && r0 + TR <= rows) {
        // every row of this thread is in range and 16-byte loadable: issue
        // all RPT loads before using any, so they are in flight together
        u32x4 raw[RPT];
#pragma unroll
        for (int rr = 0; rr < RPT; ++rr)
            raw[rr] = ld_nt<NT>(reinterpret_cast<const u32x4*>(x + (int64_t)(r0 + rg * RPT + rr) * ldx + c));
#pragma unroll
        for (int rr = 0; rr < RPT; ++rr) {
            float v[E];
            Ld<InT>::widen(raw[rr], v);
            row(rr, v);
        }
    } else {
#pragma unroll
        for (int rr = 0; rr < RPT; ++rr) {
            const int r = r0 + rg * RPT + rr;
            float v[E];
            if (r < rows && full) {
                Ld<InT>::vec(x + (int64_t)r * ldx + c, v);
            } else {
#pragma unroll
                for (int e = 0; e < E; ++e)
                    v[e] = (r < rows && c + e < cols) ? Ld<InT>::one(x + (int64_t)r * ldx + c + e) : 0.0f;
            }
            row(rr, v);
        }
    }
    if (CODES && qt) {
        // column e of this thread's chunk: RPT codes down rows rg*RPT...
        // (wcol[e][k]: rows 4k..4k+3, byte i = row 4k+i)
        uint32_t wcol[E][RPT / 4];
#pragma unroll
        for (int g = 0; g < E / 4; ++g) {
#pragma unroll
            for (int k = 0; k < RPT / 4; ++k) {
                uint32_t col[4];
                transpose4x4_bytes(codes[4 * k][g], codes[4 * k + 1][g], codes[4 * k + 2][g], codes[4 * k + 3][g],
                                   col);
#pragma unroll
                for (int j = 0; j < 4; ++j) wcol[4 * g + j][k] = col[j];
            }
        }
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const uint32_t* w = wcol[e];
            // rows rg*RPT.. of column tc+e: slot rg (8 rows) or slots 2rg,
            // 2rg+1 (16 rows, one aligned 16-byte chunk)
            uint8_t* dst = tile + tslot<E>(tc + e, rg * (RPT / 8));
            if (RPT == 16)
                *reinterpret_cast<u32x4*>(dst) = u32x4{w[0], w[1 % (RPT / 4)], w[2 % (RPT / 4)], w[3 % (RPT / 4)]};
            else
                *reinterpret_cast<u32x2*>(dst) = u32x2{w[0], w[1 % (RPT / 4)]};
        }
    }
    if (COLSUM) {
#pragma unroll
        for (int e = 0; e < E; ++e) csum[rg][tc + e] = cs[e];
    }
    __syncthreads();
    if (CODES && qt) {
        constexpr int CPC = TR / 16;  // 16-byte chunks per column
#pragma unroll
        for (int k = 0; k < kT2 * CPC / kThreads; ++k) {
            const int idx = threadIdx.x + kThreads * k;
            const int col = idx / CPC, rc = (idx % CPC) * 16;
            if (c0 + col < cols && r0 + rc < ldqt) {
                u32x4* dst = reinterpret_cast<u32x4*>(qt + (int64_t)(c0 + col) * ldqt + r0 + rc);
                const u32x4 v = *reinterpret_cast<const u32x4*>(tile + tslot<E>(col, rc >> 3));
                if (NT && qt_lines)
                    st_nt<true>(dst, v);
                else
                    st_nt<false>(dst, v);
            }
        }
    }
    if (COLSUM && r0 < rows && threadIdx.x < kT2 && c0 + threadIdx.x < cols) {
        float sum = 0.0f;
#pragma unroll
        for (int g = 0; g < RG; ++g) sum += csum[g][threadIdx.x];
        colpart[(int64_t)by * cols + c0 + threadIdx.x] = sum;
    }
    if (AMAX) {
        am = block_max_u32(am);
        if (threadIdx.x == 0) amaxpart[by * nbx + bx] = am;
    }
}

// Delayed scaling, stage 2: one block folds the tile maxima of this pass
// into its absmax, pushes it into the history (history[0] newest; the others
// move one place, the oldest drops out) and writes the scale for the next
// pass from the history's maximum (rule D1/D2).  len <= kMaxHistory.
constexpr int kMaxHistory = 1024;
__global__ __launch_bounds__(kThreads) void amax_history_kernel(const uint32_t* __restrict__ partial, int nparts,
                                                                 int fmt, float* __restrict__ history, int len,
                                                                 float* __restrict__ scale_out) {
    __shared__ uint32_t cur;
    const uint32_t m = block_max_u32(fold_parts(partial, nparts));
    if (threadIdx.x == 0) cur = m;
    constexpr int PER = kMaxHistory / kThreads;
    float old[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = threadIdx.x + k * kThreads;
        old[k] = i < len ? history[i] : 0.0f;
    }
    __syncthreads();  // every old value read, cur published
    uint32_t hm = cur;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = threadIdx.x + k * kThreads;
        if (i + 1 < len) {
            history[i + 1] = old[k];
            hm = max(hm, __float_as_uint(old[k]));
        }
    }
    if (threadIdx.x == 0) history[0] = __uint_as_float(cur);
    hm = block_max_u32(hm);
    if (threadIdx.x == 0) scale_out[0] = scale_from_absmax(__uint_as_float(hm), fmt);
}

// LayerNorm row statistics: one wave per row (4 rows per block).  Each lane
// sums its elements i = lane, lane + 64, ... in order, then a butterfly over
// the wave (every lane ends with the same bits: IEEE addition commutes).
// Two passes as in the reference (mean, then squared deviations; the second
// and third reads of the row hit the caches).  With ABSMAX the block also
// folds |y| of its rows into amaxpart[block] (the just-in-time scale of the
// fused quantize).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Rows of up to kLnRegChunks 16-byte chunks per lane (2048 bf16 or 1024
// fp32 values) stay in registers: one read of the row, 16-byte loads.
constexpr int kLnRegChunks = 4;

template <typename InT, bool ABSMAX>
__global__ __launch_bounds__(kThreads) void ln_stats_kernel(const InT* __restrict__ x, int rows, int cols, int ldx,
                                                            bool vec_ok, bool gb_vec, float eps,
                                                            const InT* __restrict__ gamma,
                                                            const InT* __restrict__ beta, float2* __restrict__ stat,
                                                            uint32_t* __restrict__ amaxpart) {
    constexpr int E = Ld<InT>::E;
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    uint32_t am = 0;
    if (r < rows && vec_ok && cols <= 64 * E * kLnRegChunks) {
        const InT* xr = x + (int64_t)r * ldx;
        const int nfull = cols / E;  // whole 16-byte chunks; the tail (< E values) is chunk nfull
        float v[kLnRegChunks][E];
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < kLnRegChunks; ++k) {
            const int j = lane + 64 * k;
            if (j < nfull) {
                Ld<InT>::vec(xr + j * E, v[k]);
            } else {
#pragma unroll
                for (int e = 0; e < E; ++e) v[k][e] = j * E + e < cols ? Ld<InT>::one(xr + j * E + e) : 0.0f;
            }
#pragma unroll
            for (int e = 0; e < E; ++e) s += v[k][e];  // padding adds +0
        }
        const float mean = wave_sum(s) / (float)cols;
        float sq = 0.0f;
#pragma unroll
        for (int k = 0; k < kLnRegChunks; ++k) {
            const int j = lane + 64 * k;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float d = v[k][e] - mean;
                sq = j * E + e < cols ? __builtin_fmaf(d, d, sq) : sq;
            }
        }
        const float var = wave_sum(sq) / (float)cols;
        const float rstd = 1.0f / __builtin_sqrtf(var + eps);
        if (lane == 0) stat[r] = make_float2(mean, rstd);
        if (ABSMAX) {
            const bool affine = gamma != nullptr;
#pragma unroll
            for (int k = 0; k < kLnRegChunks; ++k) {
                const int j = lane + 64 * k;
                float g[E], b[E];
                if (affine && gb_vec && j < nfull) {
                    Ld<InT>::vec(gamma + j * E, g);
                    Ld<InT>::vec(beta + j * E, b);
                } else {
#pragma unroll
                    for (int e = 0; e < E; ++e) {
                        const bool in = affine && j * E + e < cols;
                        g[e] = in ? Ld<InT>::one(gamma + j * E + e) : 0.0f;
                        b[e] = in ? Ld<InT>::one(beta + j * E + e) : 0.0f;
                    }
                }
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const uint32_t y = __float_as_uint(ln_apply<InT>(v[k][e], mean, rstd, affine, g[e], b[e]));
                    am = j * E + e < cols ? fold_f32(am, y) : am;
                }
            }
        }
    } else if (r < rows) {
        const InT* xr = x + (int64_t)r * ldx;
        float s = 0.0f;
        for (int i = lane; i < cols; i += 64) s += Ld<InT>::one(xr + i);
        const float mean = wave_sum(s) / (float)cols;
        float sq = 0.0f;
        for (int i = lane; i < cols; i += 64) {
            const float d = Ld<InT>::one(xr + i) - mean;
            sq = __builtin_fmaf(d, d, sq);
        }
        const float var = wave_sum(sq) / (float)cols;
        const float rstd = 1.0f / __builtin_sqrtf(var + eps);
        if (lane == 0) stat[r] = make_float2(mean, rstd);
        if (ABSMAX) {
            const bool affine = gamma != nullptr;
            for (int i = lane; i < cols; i += 64) {
                const float g = affine ? Ld<InT>::one(gamma + i) : 0.0f;
                const float b = affine ? Ld<InT>::one(beta + i) : 0.0f;
                am = fold_f32(am, __float_as_uint(ln_apply<InT>(Ld<InT>::one(xr + i), mean, rstd, affine, g, b)));
            }
        }
    }
    if (ABSMAX) {
        am = block_max_u32(am);
        if (threadIdx.x == 0) amaxpart[blockIdx.x] = am;
    }
}

// history[0..len) = amax (or 0 when amax is NULL), scale from it.
__global__ __launch_bounds__(kThreads) void amax_history_init_kernel(const float* __restrict__ amax, int fmt,
                                                                      float* __restrict__ history, int len,
                                                                      float* __restrict__ scale_out) {
    const float a = amax ? amax[0] : 0.0f;
    const float v = (a > 0.0f && a <= 3.4028234663852886e38f) ? a : 0.0f;
    for (int i = threadIdx.x; i < len; i += kThreads) history[i] = v;
    if (threadIdx.x == 0) scale_out[0] = scale_from_absmax(v, fmt);
}


// JIT: the scale comes from the absmax partials in jit (jit_block_scale;
// block (0, 0) writes absmax and scale), not from scale[0].
template <typename InT, int FMT, bool COLSUM, bool CODES, bool AMAX, bool LN, bool JIT>
__device__ __forceinline__ void q2d_kernel_body(const InT* __restrict__ x, int rows, int cols, int ldx, bool vec_ok,
                                                const float* __restrict__ scale, uint8_t* __restrict__ q, int ldq,
                                                uint8_t* __restrict__ qt, int ldqt, float* __restrict__ colpart,
                                                uint32_t* __restrict__ amaxpart, const LnArgs& ln,
                                                const JitScale& jit) {
    static_assert(!JIT || (CODES && !AMAX && !LN), "just-in-time scale: the plain code pass");
    constexpr int RG = kThreads / (kT2 / Ld<InT>::E);
    __shared__ __attribute__((aligned(16))) uint8_t tile[kT2 * kT2R];
    __shared__ float csum[COLSUM ? RG : 1][kT2];
    float sc = 1.0f;
    if constexpr (JIT)
        sc = jit_block_scale(jit.parts, jit.nparts, FMT, jit.absmax_out, jit.scale_out,
                             blockIdx.x == 0 && blockIdx.y == 0);
    else if constexpr (CODES)
        sc = scale[0];
    const QDiv d = make_qdiv(sc);
    if (!CODES || d.fast)
        q2d_tile<InT, FMT, COLSUM, CODES, AMAX, LN, true, AMAX && !LN, kT2R>(
            x, rows, cols, ldx, vec_ok, d, q, ldq, qt, ldqt, colpart, amaxpart, ln, tile, csum, blockIdx.x,
            blockIdx.y, gridDim.x);
    else
        q2d_tile<InT, FMT, COLSUM, CODES, AMAX, LN, false, AMAX && !LN, kT2R>(
            x, rows, cols, ldx, vec_ok, d, q, ldq, qt, ldqt, colpart, amaxpart, ln, tile, csum, blockIdx.x,
            blockIdx.y, gridDim.x);
}

template <typename InT, int FMT, bool COLSUM, bool CODES, bool AMAX = false, bool LN = false>
__global__ __launch_bounds__(kThreads) void quantize_2d_kernel(const InT* __restrict__ x, int rows,
                                                                int cols, int ldx, bool vec_ok,
                                                                const float* __restrict__ scale,
                                                                uint8_t* __restrict__ q, int ldq,
                                                                uint8_t* __restrict__ qt, int ldqt,
                                                                float* __restrict__ colpart,
                                                                uint32_t* __restrict__ amaxpart = nullptr,
                                                                LnArgs ln = LnArgs()) {
    q2d_kernel_body<InT, FMT, COLSUM, CODES, AMAX, LN, false>(x, rows, cols, ldx, vec_ok, scale, q, ldq, qt, ldqt,
                                                              colpart, amaxpart, ln, JitScale());
}

// The just-in-time pass (df_quantize_2d_jit), x contiguous.  The _w5 form
// holds it to five waves per SIMD, the occupancy of the same pass without the
// fold (the fold's registers are dead before the tile pass); fp32 with column
// sums has four either way and takes the plain form.
template <typename InT, int FMT, bool COLSUM>
__global__ __launch_bounds__(kThreads) void quantize_2d_jit_kernel(const InT* __restrict__ x, int rows, int cols,
                                                                    bool vec_ok, uint8_t* __restrict__ q, int ldq,
                                                                    uint8_t* __restrict__ qt, int ldqt,
                                                                    float* __restrict__ colpart, JitScale jit) {
    q2d_kernel_body<InT, FMT, COLSUM, true, false, false, true>(x, rows, cols, cols, vec_ok, nullptr, q, ldq, qt,
                                                                ldqt, colpart, nullptr, LnArgs(), jit);
}

template <typename InT, int FMT, bool COLSUM>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(5))) void quantize_2d_jit_w5_kernel(
    const InT* __restrict__ x, int rows, int cols, bool vec_ok, uint8_t* __restrict__ q, int ldq,
    uint8_t* __restrict__ qt, int ldqt, float* __restrict__ colpart, JitScale jit) {
    q2d_kernel_body<InT, FMT, COLSUM, true, false, false, true>(x, rows, cols, cols, vec_ok, nullptr, q, ldq, qt,
                                                                ldqt, colpart, nullptr, LnArgs(), jit);
}

template <typename InT, int FMT, bool COLSUM>
static void launch_q2d_jit(dim3 grid, hipStream_t st, const InT* x, int rows, int cols, bool vec_ok, uint8_t* q,
                           int ldq, uint8_t* qt, int ldqt, float* colpart, const JitScale& jit) {
    if constexpr (sizeof(InT) == 2 || !COLSUM)
        quantize_2d_jit_w5_kernel<InT, FMT, COLSUM><<<grid, kThreads, 0, st>>>(x, rows, cols, vec_ok, q, ldq, qt,
                                                                                ldqt, colpart, jit);
    else
        quantize_2d_jit_kernel<InT, FMT, COLSUM><<<grid, kThreads, 0, st>>>(x, rows, cols, vec_ok, q, ldq, qt, ldqt,
                                                                             colpart, jit);
}

// ---- several 2-D tensors in two launches (every Linear's weights after an
// optimizer step): per-tensor absmax partials, then every tensor's tiles,
// each tile block folding its tensor's partials (a launch holding an empty
// tensor runs one fold block per tensor in between).  Each tensor gets the
// same scale and codes as df_absmax_scale_* followed by df_quantize_2d
// would give it.
constexpr int kBatchMax = 32;  // tensors per launch
// Input bytes of one launch beyond which its absmax pass has pushed the
// first tensors out of the 256 MB Infinity Cache before the tile pass
// re-reads them: the tile pass then streams (non-temporal accesses).
constexpr int64_t kBatchColdBytes = (int64_t)256 << 20;

struct BatchArgs {
    int count;
    const void* x[kBatchMax];  // contiguous [rows, cols]
    int rows[kBatchMax], cols[kBatchMax];
    uint8_t* q[kBatchMax];
    uint8_t* qt[kBatchMax];
    int ldq[kBatchMax], ldqt[kBatchMax];
    int vec_ok[kBatchMax];
    int blk_first[kBatchMax + 1];   // absmax blocks of tensor t: [blk_first[t], blk_first[t+1])
    int tile_first[kBatchMax + 1];  // 2-D tiles of tensor t, row-major over tiles_x[t] columns
    int tiles_x[kBatchMax];
};

// the tensor t with first[t] <= i < first[t+1]
__device__ __forceinline__ int batch_owner(const int* first, int count, int i) {
    int lo = 0, hi = count - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (first[mid] <= i) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

template <typename InT>
__global__ __launch_bounds__(kThreads) void absmax_batch_stage1(const BatchArgs B, uint32_t* __restrict__ partial) {
    const int t = batch_owner(B.blk_first, B.count, blockIdx.x);
    const int bi = blockIdx.x - B.blk_first[t], nb = B.blk_first[t + 1] - B.blk_first[t];
    const int64_t n = (int64_t)B.rows[t] * B.cols[t];
    uint32_t m;
    if constexpr (std::is_same<InT, float>::value)
        m = absmax_f32_block(static_cast<const float*>(B.x[t]), n, bi, nb);
    else
        m = absmax_bf16_block(static_cast<const uint16_t*>(B.x[t]), n, bi, nb);
    if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

__global__ __launch_bounds__(kThreads) void absmax_batch_stage2(const BatchArgs B, const uint32_t* __restrict__ partial,
                                                                 int fmt, float* __restrict__ absmax_out,
                                                                 float* __restrict__ scale_out) {
    const int t = blockIdx.x;
    const uint32_t m = block_max_u32(fold_parts(partial + B.blk_first[t], B.blk_first[t + 1] - B.blk_first[t]));
    if (threadIdx.x == 0) {
        const float am = __uint_as_float(m);
        if (absmax_out) absmax_out[t] = am;
        scale_out[t] = scale_from_absmax(am, fmt);
    }
}

// scales from absmax values the caller supplies (df_quantize_2d_batch_absmax)
__global__ __launch_bounds__(kThreads) void scale_batch_kernel(const float* __restrict__ absmax, int count, int fmt,
                                                                float* __restrict__ scale_out) {
    for (int t = threadIdx.x; t < count; t += kThreads) scale_out[t] = scale_from_absmax(absmax[t], fmt);
}

// SRC 0: tensor t's scale is scale[t].  SRC 1: folded from its absmax
// partials, partial[blk_first[t] ..] (jit_block_scale); SRC 2: formed from
// absmax_in[t].  With SRC 1 and 2 the tensor's first tile block writes
// scale_out[t] (and absmax_out[t]).  Five waves per SIMD: the occupancy of
// the SRC 0 form (the fold's registers are dead before the tile pass).
template <typename InT, int FMT, bool NT, int SRC = 0>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(5))) void quantize_2d_batch_kernel(
    const BatchArgs B, const float* __restrict__ scale, const uint32_t* __restrict__ partial = nullptr,
    const float* __restrict__ absmax_in = nullptr, float* __restrict__ absmax_out = nullptr,
    float* __restrict__ scale_out = nullptr) {
    __shared__ __attribute__((aligned(16))) uint8_t tile[kT2 * kT2];
    __shared__ float csum[1][kT2];
    const int t = batch_owner(B.tile_first, B.count, blockIdx.x);
    const int lt = blockIdx.x - B.tile_first[t];
    const int nbx = B.tiles_x[t], bx = lt % nbx, by = lt / nbx;
    const InT* x = static_cast<const InT*>(B.x[t]);
    const int rows = B.rows[t], cols = B.cols[t];
    const bool vec_ok = B.vec_ok[t] != 0;
    float sc;
    if constexpr (SRC == 1) {
        sc = jit_block_scale(partial + B.blk_first[t], B.blk_first[t + 1] - B.blk_first[t], FMT,
                             absmax_out ? absmax_out + t : nullptr, scale_out + t, lt == 0);
    } else if constexpr (SRC == 2) {
        sc = scale_from_absmax(absmax_in[t], FMT);
        if (lt == 0 && threadIdx.x == 0) scale_out[t] = sc;
    } else {
        sc = scale[t];
    }
    const QDiv d = make_qdiv(sc);
    if (d.fast)
        q2d_tile<InT, FMT, false, true, false, false, true, NT>(x, rows, cols, cols, vec_ok, d, B.q[t], B.ldq[t], B.qt[t],
                                                            B.ldqt[t], nullptr, nullptr, LnArgs(), tile, csum, bx, by,
                                                            nbx);
    else
        q2d_tile<InT, FMT, false, true, false, false, false, NT>(x, rows, cols, cols, vec_ok, d, B.q[t], B.ldq[t],
                                                             B.qt[t], B.ldqt[t], nullptr, nullptr, LnArgs(), tile,
                                                             csum, bx, by, nbx);
}

// out[c] = sum over tile rows of colpart[t][c].  A block owns 64 columns;
// its 4 waves each take every 4th tile row (8 independent loads in flight
// per thread), then the 4 partial sums are added in wave order -- the same
// order on every run.
__global__ __launch_bounds__(kThreads) void colsum_reduce_kernel(const float* __restrict__ colpart,
                                                                  int tiles, int cols,
                                                                  float* __restrict__ out) {
    __shared__ float part[4][64];
    const int c = blockIdx.x * 64 + (threadIdx.x & 63);
    const int w = threadIdx.x >> 6;
    float s = 0.0f;
    if (c < cols) {
        int t = w;
        for (; t + 28 < tiles; t += 32) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = colpart[(int64_t)(t + 4 * u) * cols + c];
#pragma unroll
            for (int u = 0; u < 8; ++u) s += v[u];
        }
        for (; t < tiles; t += 4) s += colpart[(int64_t)t * cols + c];
    }
    part[w][threadIdx.x & 63] = s;
    __syncthreads();
    if (w == 0 && c < cols)
        out[c] = ((part[0][threadIdx.x] + part[1][threadIdx.x]) + part[2][threadIdx.x]) + part[3][threadIdx.x];
}

// ------------------------------------------------------ bandwidth probe --
// The flat kernels' access pattern without their arithmetic: per chunk,
// each thread issues U non-temporal loads of RB bytes, kThreads apart,
// then U non-temporal stores of WB bytes at the same vector index (the
// stored words are an XOR fold of the loaded ones, so no load is dead); U
// is the depth of the kernel with that pattern (kU for the read, kUQuant*
// and kUDeq* for the conversions, kUDeqF32 for the copy).
// RB:WB = 16:4 is fp32 -> fp8, 16:8 bf16 -> fp8, 4:16 fp8 -> fp32, 8:16
// fp8 -> bf16, 16:16 a copy, 16:0 a read (absmax: one word per block).
template <int RB> struct ProbeVec;
template <> struct ProbeVec<4> { using T = uint32_t; };
template <> struct ProbeVec<8> { using T = u32x2; };
template <> struct ProbeVec<16> { using T = u32x4; };

__device__ __forceinline__ uint32_t fold_words(uint32_t v) { return v; }
__device__ __forceinline__ uint32_t fold_words(u32x2 v) { return v.x ^ v.y; }
__device__ __forceinline__ uint32_t fold_words(u32x4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

template <int WB> struct ProbeOut;
template <> struct ProbeOut<4> {
    template <typename V> static __device__ __forceinline__ uint32_t make(V v) { return fold_words(v); }
};
template <> struct ProbeOut<8> {
    static __device__ __forceinline__ u32x2 make(u32x4 v) { return u32x2{v.x ^ v.y, v.z ^ v.w}; }
};
template <> struct ProbeOut<16> {
    static __device__ __forceinline__ u32x4 make(uint32_t w) { return u32x4{w, w ^ 1u, w ^ 2u, w ^ 3u}; }
    static __device__ __forceinline__ u32x4 make(u32x2 w) { return u32x4{w.x, w.y, w.x ^ 1u, w.y ^ 1u}; }
    static __device__ __forceinline__ u32x4 make(u32x4 v) { return u32x4{v.x ^ 1u, v.y, v.z, v.w}; }
};

template <int RB, int WB, int U>
__global__ __launch_bounds__(kThreads) void hbm_probe_kernel(const void* __restrict__ src, int64_t nvec,
                                                               void* __restrict__ dst) {
    using V = typename ProbeVec<RB>::T;
    const V* xv = reinterpret_cast<const V*>(src);
    constexpr int64_t CH = (int64_t)kThreads * U;
    uint32_t acc = 0;
    for (int64_t base = (int64_t)blockIdx.x * CH; base < nvec; base += (int64_t)gridDim.x * CH) {
        V v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(xv + base + u * kThreads + threadIdx.x);
        if constexpr (WB == 0) {
#pragma unroll
            for (int u = 0; u < U; ++u) acc ^= fold_words(v[u]);
        } else {
            using O = decltype(ProbeOut<WB>::make(v[0]));
            O* ov = reinterpret_cast<O*>(dst);
#pragma unroll
            for (int u = 0; u < U; ++u)
                __builtin_nontemporal_store(ProbeOut<WB>::make(v[u]), ov + base + u * kThreads + threadIdx.x);
        }
    }
    if constexpr (WB == 0) {
        const uint32_t m = block_max_u32(acc);
        if (threadIdx.x == 0) reinterpret_cast<uint32_t*>(dst)[blockIdx.x] = m;
    }
}

// --------------------------------------------------------------- launchers --
static int grid_for(int64_t units, int64_t per_block_unit_cap) {
    int64_t blocks = (units + kThreads - 1) / kThreads;
    if (blocks > per_block_unit_cap) blocks = per_block_unit_cap;
    return blocks < 1 ? 1 : (int)blocks;
}

}  // namespace dfk

using namespace dfk;

// Grid cap for the quantize/dequantize kernels: one chunk per block up to
// 2^28 elements, grid-stride beyond.  Many short-lived blocks keep more of
// the chip's store traffic in flight than 2048 looping blocks: +5-7% at
// config 2 (e.g. fp32 -> e4m3 5.52-5.65 -> 5.91-6.01 TB/s with 8 vectors
// per thread).
static constexpr int64_t kStreamBlocks = 131072;

// blocks for n elements, per elements per thread vector, U vectors per thread
static int stream_grid(int64_t n, int per, int U) {
    return grid_for((n / per + 1 + U - 1) / U, kStreamBlocks);
}

extern "C" size_t df_absmax_workspace_bytes(void) { return kMaxReduceBlocks * sizeof(uint32_t); }

extern "C" size_t df_hbm_probe_dst_bytes(int read_bytes, int write_bytes, int64_t src_bytes) {
    if (read_bytes <= 0 || src_bytes <= 0) return 0;
    const int64_t nvec = src_bytes / read_bytes;
    if (write_bytes == 0) return (size_t)grid_for(nvec / kU, kStreamBlocks) * sizeof(uint32_t);
    return (size_t)(nvec * write_bytes);
}

extern "C" int df_hbm_probe(int read_bytes, int write_bytes, const void* src, int64_t src_bytes, void* dst,
                            void* stream) {
    clear_error();
    static const char* name = "df_hbm_probe";
    const bool ok = (read_bytes == 16 && (write_bytes == 0 || write_bytes == 4 || write_bytes == 8 ||
                                          write_bytes == 16)) ||
                    ((read_bytes == 4 || read_bytes == 8) && write_bytes == 16);
    DF_CHECK(ok, DF_ERR_UNSUPPORTED, "%s: pattern %d:%d not provided", name, read_bytes, write_bytes);
    DF_CHECK(src && dst, DF_ERR_INVALID, "%s: NULL pointer", name);
    const int U = read_bytes == 16 ? (write_bytes == 0 ? kU : write_bytes == 4 ? kUQuantF32
                                                          : write_bytes == 8 ? kUQuantBf16 : kUDeqF32)
                                    : (read_bytes == 4 ? kUDeqF32 : kUDeqBf16);
    const int64_t chunk_bytes = (int64_t)kThreads * U * read_bytes;
    DF_CHECK(src_bytes > 0 && src_bytes % chunk_bytes == 0, DF_ERR_INVALID,
             "%s: src_bytes=%lld must be a positive multiple of %lld", name, (long long)src_bytes,
             (long long)chunk_bytes);
    DF_CHECK(aligned16(src) && aligned16(dst), DF_ERR_ALIGN, "%s: src and dst must be 16-byte aligned", name);
    const int64_t nvec = src_bytes / read_bytes;
    const int blocks = grid_for(nvec / U, kStreamBlocks);
    hipStream_t st = as_stream(stream);
#define DF_PROBE(R, W, UU)                                                             \
    if (read_bytes == R && write_bytes == W) {                                         \
        hbm_probe_kernel<R, W, UU><<<blocks, kThreads, 0, st>>>(src, nvec, dst);      \
        return launch_status(name);                                                    \
    }
    DF_PROBE(16, 0, kU)
    DF_PROBE(16, 4, kUQuantF32)
    DF_PROBE(16, 8, kUQuantBf16)
    DF_PROBE(16, 16, kUDeqF32)
    DF_PROBE(4, 16, kUDeqF32)
    DF_PROBE(8, 16, kUDeqBf16)
#undef DF_PROBE
    return DF_ERR_UNSUPPORTED;
}

// One partial maximum per block into part[0 .. blocks), blocks <= cap <=
// kMaxReduceBlocks (x 16-byte aligned, dtype already checked); returns blocks.
static int launch_absmax_stage1(int in_dtype, const void* x, int64_t n, uint32_t* part, hipStream_t st,
                                int cap = kMaxReduceBlocks) {
    const int per = in_dtype == DF_DTYPE_FLOAT32 ? 4 : 8;
    const int blocks = grid_for((n / per + kU - 1) / kU, cap);
    if (in_dtype == DF_DTYPE_FLOAT32)
        absmax_f32_stage1<<<blocks, kThreads, 0, st>>>(static_cast<const float*>(x), n, part);
    else if (in_dtype == DF_DTYPE_BFLOAT16)
        absmax_bf16_stage1<<<blocks, kThreads, 0, st>>>(static_cast<const uint16_t*>(x), n, part);
    else
        absmax_f16_stage1<<<blocks, kThreads, 0, st>>>(static_cast<const uint16_t*>(x), n, part);
    return blocks;
}

static int absmax_impl(int in_dtype, const void* x, int64_t n, int fmt, float* absmax_dev,
                       float* scale_dev, void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    DF_CHECK(n >= 0, DF_ERR_INVALID, "absmax: n < 0");
    DF_CHECK(x || n == 0, DF_ERR_INVALID, "absmax: x is NULL");
    DF_CHECK(absmax_dev || scale_dev, DF_ERR_INVALID, "absmax: no output");
    DF_CHECK(ws, DF_ERR_WORKSPACE, "absmax: workspace is NULL");
    DF_CHECK(ws_bytes >= df_absmax_workspace_bytes(), DF_ERR_WORKSPACE,
             "absmax: workspace %zu bytes < %zu", ws_bytes, df_absmax_workspace_bytes());
    DF_CHECK(fmt == E4M3 || fmt == E5M2, DF_ERR_UNSUPPORTED, "absmax: bad fp8 format %d", fmt);
    DF_CHECK(aligned16(x) && aligned4(ws), DF_ERR_ALIGN, "absmax: x must be 16-byte aligned");
    DF_CHECK(in_dtype == DF_DTYPE_FLOAT32 || in_dtype == DF_DTYPE_BFLOAT16 || in_dtype == DF_DTYPE_HALF,
             DF_ERR_UNSUPPORTED, "absmax: dtype %d not supported", in_dtype);
    hipStream_t st = as_stream(stream);
    uint32_t* part = static_cast<uint32_t*>(ws);
    const int blocks = launch_absmax_stage1(in_dtype, x, n, part, st);
    absmax_stage2<<<1, kThreads, 0, st>>>(part, blocks, fmt, absmax_dev, scale_dev);
    return launch_status("absmax");
}

extern "C" int df_absmax_f32(const float* x, int64_t n, float* absmax_dev, void* ws,
                             size_t ws_bytes, void* stream) {
    DF_CHECK(absmax_dev, DF_ERR_INVALID, "df_absmax_f32: absmax_dev is NULL");
    return absmax_impl(DF_DTYPE_FLOAT32, x, n, E4M3, absmax_dev, nullptr, ws, ws_bytes, stream);
}
extern "C" int df_absmax_bf16(const uint16_t* x, int64_t n, float* absmax_dev, void* ws,
                              size_t ws_bytes, void* stream) {
    DF_CHECK(absmax_dev, DF_ERR_INVALID, "df_absmax_bf16: absmax_dev is NULL");
    return absmax_impl(DF_DTYPE_BFLOAT16, x, n, E4M3, absmax_dev, nullptr, ws, ws_bytes, stream);
}
extern "C" int df_absmax_f16(const uint16_t* x, int64_t n, float* absmax_dev, void* ws,
                             size_t ws_bytes, void* stream) {
    DF_CHECK(absmax_dev, DF_ERR_INVALID, "df_absmax_f16: absmax_dev is NULL");
    return absmax_impl(DF_DTYPE_HALF, x, n, E4M3, absmax_dev, nullptr, ws, ws_bytes, stream);
}
extern "C" int df_absmax_scale_f32(const float* x, int64_t n, int fmt, float* absmax_dev,
                                   float* scale_dev, void* ws, size_t ws_bytes, void* stream) {
    return absmax_impl(DF_DTYPE_FLOAT32, x, n, fmt, absmax_dev, scale_dev, ws, ws_bytes, stream);
}
extern "C" int df_absmax_scale_bf16(const uint16_t* x, int64_t n, int fmt, float* absmax_dev,
                                    float* scale_dev, void* ws, size_t ws_bytes, void* stream) {
    return absmax_impl(DF_DTYPE_BFLOAT16, x, n, fmt, absmax_dev, scale_dev, ws, ws_bytes, stream);
}
extern "C" int df_absmax_scale_f16(const uint16_t* x, int64_t n, int fmt, float* absmax_dev,
                                   float* scale_dev, void* ws, size_t ws_bytes, void* stream) {
    return absmax_impl(DF_DTYPE_HALF, x, n, fmt, absmax_dev, scale_dev, ws, ws_bytes, stream);
}

extern "C" int df_compute_scale(const float* absmax_dev, int fmt, float* scale_dev, void* stream) {
    clear_error();
    DF_CHECK(absmax_dev && scale_dev, DF_ERR_INVALID, "df_compute_scale: NULL pointer");
    DF_CHECK(fmt == E4M3 || fmt == E5M2, DF_ERR_UNSUPPORTED, "df_compute_scale: bad format %d", fmt);
    scale_kernel<<<1, 64, 0, as_stream(stream)>>>(absmax_dev, fmt, scale_dev);
    return launch_status("df_compute_scale");
}

template <int FMT>
static int quantize_f32_impl(const float* x, int64_t n, const float* scale, uint8_t* q, void* stream,
                             const char* name) {
    clear_error();
    DF_CHECK(n >= 0, DF_ERR_INVALID, "%s: n < 0", name);
    if (n == 0) return DF_OK;
    DF_CHECK(x && scale && q, DF_ERR_INVALID, "%s: NULL pointer", name);
    DF_CHECK(aligned16(x) && aligned4(q), DF_ERR_ALIGN, "%s: x must be 16-byte and q 4-byte aligned", name);
    const int blocks = stream_grid(n, 4, kUQuantF32);
    if (aligned128(q))
        quantize_f32_kernel<FMT, true><<<blocks, kThreads, 0, as_stream(stream)>>>(x, n, scale, q);
    else
        quantize_f32_kernel<FMT, false><<<blocks, kThreads, 0, as_stream(stream)>>>(x, n, scale, q);
    return launch_status(name);
}

template <int FMT>
static int quantize_bf16_impl(const uint16_t* x, int64_t n, const float* scale, uint8_t* q,
                              void* stream, const char* name) {
    clear_error();
    DF_CHECK(n >= 0, DF_ERR_INVALID, "%s: n < 0", name);
    if (n == 0) return DF_OK;
    DF_CHECK(x && scale && q, DF_ERR_INVALID, "%s: NULL pointer", name);
    DF_CHECK(aligned16(x) && (((uintptr_t)q & 7u) == 0), DF_ERR_ALIGN,
             "%s: x must be 16-byte and q 8-byte aligned", name);
    const int blocks = stream_grid(n, 8, kUQuantBf16);
    if (aligned128(q))
        quantize_bf16_kernel<FMT, true><<<blocks, kThreads, 0, as_stream(stream)>>>(x, n, scale, q);
    else
        quantize_bf16_kernel<FMT, false><<<blocks, kThreads, 0, as_stream(stream)>>>(x, n, scale, q);
    return launch_status(name);
}

extern "C" int df_quantize_f32_e4m3(const float* x, int64_t n, const float* s, uint8_t* q, void* st) {
    return quantize_f32_impl<E4M3>(x, n, s, q, st, "df_quantize_f32_e4m3");
}
extern "C" int df_quantize_f32_e5m2(const float* x, int64_t n, const float* s, uint8_t* q, void* st) {
    return quantize_f32_impl<E5M2>(x, n, s, q, st, "df_quantize_f32_e5m2");
}
extern "C" int df_quantize_bf16_e4m3(const uint16_t* x, int64_t n, const float* s, uint8_t* q, void* st) {
    return quantize_bf16_impl<E4M3>(x, n, s, q, st, "df_quantize_bf16_e4m3");
}
extern "C" int df_quantize_bf16_e5m2(const uint16_t* x, int64_t n, const float* s, uint8_t* q, void* st) {
    return quantize_bf16_impl<E5M2>(x, n, s, q, st, "df_quantize_bf16_e5m2");
}

template <int FMT>
static int dequantize_f32_impl(const uint8_t* q, int64_t n, const float* scale, float* out,
                               void* stream, const char* name) {
    clear_error();
    DF_CHECK(n >= 0, DF_ERR_INVALID, "%s: n < 0", name);
    if (n == 0) return DF_OK;
    DF_CHECK(q && scale && out, DF_ERR_INVALID, "%s: NULL pointer", name);
    DF_CHECK(aligned4(q) && aligned16(out), DF_ERR_ALIGN, "%s: q must be 4-byte and out 16-byte aligned",
             name);
    const int blocks = stream_grid(n, 4, kUDeqF32);
    if (aligned128(out))
        dequantize_f32_kernel<FMT, true><<<blocks, kThreads, 0, as_stream(stream)>>>(q, n, scale, out);
    else
        dequantize_f32_kernel<FMT, false><<<blocks, kThreads, 0, as_stream(stream)>>>(q, n, scale, out);
    return launch_status(name);
}

template <int FMT>
static int dequantize_bf16_impl(const uint8_t* q, int64_t n, const float* scale, uint16_t* out,
                                void* stream, const char* name) {
    clear_error();
    DF_CHECK(n >= 0, DF_ERR_INVALID, "%s: n < 0", name);
    if (n == 0) return DF_OK;
    DF_CHECK(q && scale && out, DF_ERR_INVALID, "%s: NULL pointer", name);
    DF_CHECK((((uintptr_t)q & 7u) == 0) && aligned16(out), DF_ERR_ALIGN,
             "%s: q must be 8-byte and out 16-byte aligned", name);
    const int blocks = stream_grid(n, 8, kUDeqBf16);
    if (aligned128(out))
        dequantize_bf16_kernel<FMT, true><<<blocks, kThreads, 0, as_stream(stream)>>>(q, n, scale, out);
    else
        dequantize_bf16_kernel<FMT, false><<<blocks, kThreads, 0, as_stream(stream)>>>(q, n, scale, out);
    return launch_status(name);
}

extern "C" int df_dequantize_e4m3_f32(const uint8_t* q, int64_t n, const float* s, float* o, void* st) {
    return dequantize_f32_impl<E4M3>(q, n, s, o, st, "df_dequantize_e4m3_f32");
}
extern "C" int df_dequantize_e5m2_f32(const uint8_t* q, int64_t n, const float* s, float* o, void* st) {
    return dequantize_f32_impl<E5M2>(q, n, s, o, st, "df_dequantize_e5m2_f32");
}
extern "C" int df_dequantize_e4m3_bf16(const uint8_t* q, int64_t n, const float* s, uint16_t* o, void* st) {
    return dequantize_bf16_impl<E4M3>(q, n, s, o, st, "df_dequantize_e4m3_bf16");
}
extern "C" int df_dequantize_e5m2_bf16(const uint8_t* q, int64_t n, const float* s, uint16_t* o, void* st) {
    return dequantize_bf16_impl<E5M2>(q, n, s, o, st, "df_dequantize_e5m2_bf16");
}

extern "C" size_t df_quantize_2d_workspace_bytes(int rows, int cols) {
    if (rows <= 0 || cols <= 0) return 0;
    return (size_t)((rows + kT2R - 1) / kT2R) * (size_t)cols * sizeof(float);
}

// df_quantize_2d_jit's workspace: the column-sum partials (when asked), then
// the absmax partials at *parts_off (16-byte aligned).
static size_t jit_ws_layout(int rows, int cols, bool colsum, size_t* parts_off) {
    const size_t cs = colsum ? (df_quantize_2d_workspace_bytes(rows, cols) + 15) & ~(size_t)15 : 0;
    if (parts_off) *parts_off = cs;
    return cs + kMaxReduceBlocks * sizeof(uint32_t);
}

extern "C" size_t df_quantize_2d_jit_workspace_bytes(int rows, int cols, int colsum) {
    if (rows < 0 || cols < 0) return 0;
    return jit_ws_layout(rows, cols, colsum != 0, nullptr);
}

// Tile grid of a 2-D quantize (tiles of tr rows and kT2 columns): covers the
// codes' padded extents.
static dim3 q2d_grid(int rows, int cols, const uint8_t* q, int ldq, const uint8_t* qt, int ldqt, int tr) {
    const int row_ext = qt ? (rows > ldqt ? rows : ldqt) : rows;
    const int col_ext = q ? (cols > ldq ? cols : ldq) : cols;
    return dim3((col_ext + kT2 - 1) / kT2, (row_ext + tr - 1) / tr);
}

// Delayed-scaling workspace: column-sum partials (when asked for), then one
// tile maximum per block, 16-byte aligned.
static size_t delayed_ws_layout(int rows, int cols, int ldq, int ldqt, bool colsum, size_t* amax_off) {
    const size_t cs = colsum ? df_quantize_2d_workspace_bytes(rows, cols) : 0;
    const size_t off = (cs + 15) & ~(size_t)15;
    const dim3 g = q2d_grid(rows, cols, (const uint8_t*)1, ldq, ldqt > 0 ? (const uint8_t*)1 : nullptr, ldqt, kT2R);
    if (amax_off) *amax_off = off;
    return off + (size_t)g.x * g.y * sizeof(uint32_t);
}

static int quantize_2d_impl(const char* name, int in_dtype, const void* x, int rows, int cols, int ldx,
                            int fmt, const float* scale_dev, uint8_t* q, int ldq, uint8_t* qt, int ldqt,
                            float* colsum, void* ws, size_t ws_bytes, void* stream,
                            float* history = nullptr, int hist_len = 0, float* next_scale = nullptr,
                            bool jit = false, float* jit_absmax = nullptr) {
    clear_error();
    DF_CHECK(rows >= 0 && cols >= 0 && (ldx >= cols || rows == 0), DF_ERR_INVALID,
             "%s: bad shape rows=%d cols=%d ldx=%d", name, rows, cols, ldx);
    const bool empty = rows == 0 || cols == 0;  // nothing to write: outputs may be NULL
    DF_CHECK(q || qt || colsum || empty, DF_ERR_INVALID, "%s: no output", name);
    DF_CHECK((scale_dev || (!q && !qt)) && (x || rows * (int64_t)cols == 0), DF_ERR_INVALID, "%s: NULL pointer", name);
    DF_CHECK(fmt == E4M3 || fmt == E5M2, DF_ERR_UNSUPPORTED, "%s: bad format %d", name, fmt);
    DF_CHECK(in_dtype == DF_DTYPE_FLOAT32 || in_dtype == DF_DTYPE_BFLOAT16 || in_dtype == DF_DTYPE_HALF,
             DF_ERR_UNSUPPORTED, "%s: dtype %d not supported", name, in_dtype);
    if (q) {
        DF_CHECK(ldq >= cols && ldq % 16 == 0, DF_ERR_ALIGN, "%s: ldq=%d must be >= cols and a multiple of 16", name, ldq);
        DF_CHECK(aligned16(q), DF_ERR_ALIGN, "%s: q must be 16-byte aligned", name);
    }
    if (qt) {
        DF_CHECK(ldqt >= rows && ldqt % 16 == 0, DF_ERR_ALIGN, "%s: ldqt=%d must be >= rows and a multiple of 16", name, ldqt);
        DF_CHECK(aligned16(qt), DF_ERR_ALIGN, "%s: qt must be 16-byte aligned", name);
    }
    const bool delayed = history != nullptr;
    size_t amax_off = 0, jit_off = 0;
    if (jit) {  // scale_dev is an output here
        DF_CHECK(q || qt || empty, DF_ERR_INVALID, "%s: no code output", name);
        DF_CHECK(ldx == cols, DF_ERR_INVALID, "%s: x must be contiguous (ldx=%d, cols=%d)", name, ldx, cols);
        DF_CHECK(aligned4(scale_dev) && aligned4(jit_absmax), DF_ERR_ALIGN, "%s: absmax/scale misaligned", name);
        DF_CHECK(aligned16(x), DF_ERR_ALIGN, "%s: x must be 16-byte aligned", name);
        const size_t need = jit_ws_layout(rows, cols, colsum != nullptr, &jit_off);
        DF_CHECK(ws && aligned16(ws), DF_ERR_WORKSPACE, "%s: needs a 16-byte aligned workspace", name);
        DF_CHECK(ws_bytes >= need, DF_ERR_WORKSPACE, "%s: workspace %zu bytes < %zu", name, ws_bytes, need);
    } else if (delayed) {
        DF_CHECK(q || qt || empty, DF_ERR_INVALID, "%s: no code output", name);
        DF_CHECK(hist_len >= 1 && hist_len <= kMaxHistory, DF_ERR_INVALID, "%s: history length %d not in [1, %d]",
                 name, hist_len, kMaxHistory);
        DF_CHECK(aligned4(history) && aligned4(next_scale), DF_ERR_ALIGN, "%s: history/scale misaligned", name);
        const size_t need = delayed_ws_layout(rows, cols, q ? ldq : 0, qt ? ldqt : 0, colsum != nullptr, &amax_off);
        DF_CHECK(ws && aligned16(ws), DF_ERR_WORKSPACE, "%s: needs a 16-byte aligned workspace", name);
        DF_CHECK(ws_bytes >= need, DF_ERR_WORKSPACE, "%s: workspace %zu bytes < %zu", name, ws_bytes, need);
    } else if (colsum) {
        DF_CHECK(ws && aligned4(ws), DF_ERR_WORKSPACE, "%s: column sums need a workspace", name);
        DF_CHECK(ws_bytes >= df_quantize_2d_workspace_bytes(rows, cols), DF_ERR_WORKSPACE,
                 "%s: workspace %zu bytes < %zu", name, ws_bytes, df_quantize_2d_workspace_bytes(rows, cols));
    }
    const dim3 grid = q2d_grid(rows, cols, q, ldq, qt, ldqt, kT2R);
    hipStream_t st = as_stream(stream);
    if (grid.x == 0 || grid.y == 0) {
        if (colsum && cols > 0) {
            const float zero = 0.0f;
            if (int rc = df_fill(colsum, cols, 4, &zero, stream)) return rc;
        }
        if (delayed) {  // an empty pass measures absmax 0
            amax_history_kernel<<<1, kThreads, 0, st>>>(nullptr, 0, fmt, history, hist_len, next_scale);
            return launch_status(name);
        }
        if (jit) {  // absmax 0, scale 1
            absmax_stage2<<<1, kThreads, 0, st>>>(nullptr, 0, fmt, jit_absmax, const_cast<float*>(scale_dev));
            return launch_status(name);
        }
        return DF_OK;
    }
    DF_CHECK(grid.y <= 65535, DF_ERR_INVALID, "%s: rows=%d too large", name, rows);
    float* part = colsum ? static_cast<float*>(ws) : nullptr;
    uint32_t* amaxpart = delayed ? reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + amax_off) : nullptr;
    const int esz = in_dtype == DF_DTYPE_FLOAT32 ? 4 : 2;
    const bool vec_ok = aligned16(x) && ((int64_t)ldx * esz) % 16 == 0;
    JitScale J;
    if (jit) {
        uint32_t* jparts = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + jit_off);
        J.nparts = launch_absmax_stage1(in_dtype, x, (int64_t)rows * cols, jparts, st, kJitParts);
        J.parts = jparts;
        J.absmax_out = jit_absmax;
        J.scale_out = const_cast<float*>(scale_dev);
    }
#define DF_Q2D(T, F, CS)                                                                                        \
    do {                                                                                                        \
        if (jit)                                                                                                \
            launch_q2d_jit<T, F, CS>(grid, st, static_cast<const T*>(x), rows, cols, vec_ok, q, ldq, qt, ldqt,   \
                                     part, J);                                                                  \
        else if (delayed)                                                                                       \
            quantize_2d_kernel<T, F, CS, true, true><<<grid, kThreads, 0, st>>>(                                \
                static_cast<const T*>(x), rows, cols, ldx, vec_ok, scale_dev, q, ldq, qt, ldqt, part, amaxpart); \
        else                                                                                                    \
            quantize_2d_kernel<T, F, CS, true><<<grid, kThreads, 0, st>>>(                                      \
                static_cast<const T*>(x), rows, cols, ldx, vec_ok, scale_dev, q, ldq, qt, ldqt, part);          \
    } while (0)
    if (!q && !qt) {  // column sums only
        if (in_dtype == DF_DTYPE_FLOAT32)
            quantize_2d_kernel<float, E4M3, true, false><<<grid, kThreads, 0, st>>>(
                static_cast<const float*>(x), rows, cols, ldx, vec_ok, nullptr, nullptr, 0, nullptr, 0, part);
        else if (in_dtype == DF_DTYPE_HALF)
            quantize_2d_kernel<f16_t, E4M3, true, false><<<grid, kThreads, 0, st>>>(
                static_cast<const f16_t*>(x), rows, cols, ldx, vec_ok, nullptr, nullptr, 0, nullptr, 0, part);
        else
            quantize_2d_kernel<uint16_t, E4M3, true, false><<<grid, kThreads, 0, st>>>(
                static_cast<const uint16_t*>(x), rows, cols, ldx, vec_ok, nullptr, nullptr, 0, nullptr, 0, part);
    } else if (in_dtype == DF_DTYPE_FLOAT32) {
        if (fmt == E4M3) { if (colsum) DF_Q2D(float, E4M3, true); else DF_Q2D(float, E4M3, false); }
        else { if (colsum) DF_Q2D(float, E5M2, true); else DF_Q2D(float, E5M2, false); }
    } else if (in_dtype == DF_DTYPE_HALF) {
        if (fmt == E4M3) { if (colsum) DF_Q2D(f16_t, E4M3, true); else DF_Q2D(f16_t, E4M3, false); }
        else { if (colsum) DF_Q2D(f16_t, E5M2, true); else DF_Q2D(f16_t, E5M2, false); }
    } else {
        if (fmt == E4M3) { if (colsum) DF_Q2D(uint16_t, E4M3, true); else DF_Q2D(uint16_t, E4M3, false); }
        else { if (colsum) DF_Q2D(uint16_t, E5M2, true); else DF_Q2D(uint16_t, E5M2, false); }
    }
#undef DF_Q2D
    if (colsum)
        colsum_reduce_kernel<<<(cols + 63) / 64, kThreads, 0, st>>>(part, rows == 0 ? 0 : (rows + kT2R - 1) / kT2R,
                                                                    cols, colsum);
    if (delayed)
        amax_history_kernel<<<1, kThreads, 0, st>>>(amaxpart, (int)(grid.x * grid.y), fmt, history, hist_len,
                                                    next_scale);
    return launch_status(name);
}

extern "C" int df_amax_history_init(const float* amax_dev, int fmt, float* history, int len, float* scale_dev,
                                    void* stream) {
    clear_error();
    DF_CHECK(history && scale_dev, DF_ERR_INVALID, "df_amax_history_init: NULL pointer");
    DF_CHECK(len >= 1 && len <= kMaxHistory, DF_ERR_INVALID, "df_amax_history_init: length %d not in [1, %d]", len,
             kMaxHistory);
    DF_CHECK(fmt == E4M3 || fmt == E5M2, DF_ERR_UNSUPPORTED, "df_amax_history_init: bad format %d", fmt);
    DF_CHECK(aligned4(history) && aligned4(scale_dev) && (!amax_dev || aligned4(amax_dev)), DF_ERR_ALIGN,
             "df_amax_history_init: misaligned pointer");
    amax_history_init_kernel<<<1, kThreads, 0, as_stream(stream)>>>(amax_dev, fmt, history, len, scale_dev);
    return launch_status("df_amax_history_init");
}

extern "C" size_t df_quantize_2d_delayed_workspace_bytes(int rows, int cols, int ldq, int ldqt, int colsum) {
    if (rows < 0 || cols < 0) return 0;
    return delayed_ws_layout(rows, cols, ldq, ldqt, colsum != 0, nullptr);
}

extern "C" int df_quantize_2d_delayed(int in_dtype, const void* x, int rows, int cols, int ldx, int fmt,
                                      const float* scale_dev, float* next_scale_dev, float* history, int len,
                                      uint8_t* q, int ldq, uint8_t* qt, int ldqt, float* colsum, void* ws,
                                      size_t ws_bytes, void* stream) {
    DF_CHECK(history && scale_dev && next_scale_dev, DF_ERR_INVALID, "df_quantize_2d_delayed: NULL pointer");
    return quantize_2d_impl("df_quantize_2d_delayed", in_dtype, x, rows, cols, ldx, fmt, scale_dev, q, ldq, qt,
                            ldqt, colsum, ws, ws_bytes, stream, history, len, next_scale_dev);
}

// ---- allocation-free delayed-scaling quantize -----------------------------
// The workspace of df_quantize_2d_delayed (column-sum partials, then one
// tile maximum per block) lives in this file-scope device array instead of a
// caller's buffer.  Every block overwrites its own entries before the fold
// kernels read them, so nothing in it has to start at zero.  Each GPU holds
// its own copy at its own address; host code uses only the address that
// hipGetSymbolAddress returns for the current device (the array's name on
// the host is a stand-in, not a device address).
constexpr size_t kNoAllocScratchBytes = DF_QUANTIZE_2D_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

// The current device's address of `scratch`, looked up on the first call on
// that device; nullptr (and the error message set) on failure.
static void* scratch_for_current_device(const char* name) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_error("%s: no current device (or device index %d beyond %d)", name, dev, kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            set_error("%s: hipGetSymbolAddress(scratch) on device %d: %s", name, dev, hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}

extern "C" int df_quantize_2d_delayed_noalloc(int in_dtype, const void* x, int rows, int cols, int ldx, int fmt,
                                              const float* scale_dev, float* next_scale_dev, float* history, int len,
                                              uint8_t* q, int ldq, uint8_t* qt, int ldqt, float* colsum,
                                              void* stream) {
    clear_error();
    static const char* name = "df_quantize_2d_delayed_noalloc";
    DF_CHECK(history && scale_dev && next_scale_dev, DF_ERR_INVALID, "%s: NULL pointer", name);
    DF_CHECK(rows >= 0 && cols >= 0, DF_ERR_INVALID, "%s: bad shape rows=%d cols=%d", name, rows, cols);
    const size_t need = delayed_ws_layout(rows, cols, q ? ldq : 0, qt ? ldqt : 0, colsum != nullptr, nullptr);
    DF_CHECK(need <= kNoAllocScratchBytes, DF_ERR_WORKSPACE,
             "%s: rows=%d cols=%d need %zu bytes of scratch, above this entry point's fixed %zu bytes "
             "(use df_quantize_2d_delayed with a workspace)",
             name, rows, cols, need, kNoAllocScratchBytes);
    void* ws = scratch_for_current_device(name);
    if (!ws) return DF_ERR_HIP;
    return quantize_2d_impl(name, in_dtype, x, rows, cols, ldx, fmt, scale_dev, q, ldq, qt, ldqt, colsum, ws,
                            kNoAllocScratchBytes, stream, history, len, next_scale_dev);
}

extern "C" int df_quantize_2d(int in_dtype, const void* x, int rows, int cols, int ldx, int fmt,
                              const float* scale_dev, uint8_t* q, int ldq, uint8_t* qt, int ldqt,
                              void* stream) {
    DF_CHECK(q || qt || rows == 0 || cols == 0, DF_ERR_INVALID, "df_quantize_2d: no output");
    return quantize_2d_impl("df_quantize_2d", in_dtype, x, rows, cols, ldx, fmt, scale_dev, q, ldq, qt, ldqt,
                            nullptr, nullptr, 0, stream);
}

extern "C" int df_quantize_2d_colsum(int in_dtype, const void* x, int rows, int cols, int ldx, int fmt,
                                     const float* scale_dev, uint8_t* q, int ldq, uint8_t* qt, int ldqt,
                                     float* colsum, void* ws, size_t ws_bytes, void* stream) {
    DF_CHECK(colsum, DF_ERR_INVALID, "df_quantize_2d_colsum: colsum is NULL");
    return quantize_2d_impl("df_quantize_2d_colsum", in_dtype, x, rows, cols, ldx, fmt, scale_dev, q, ldq, qt,
                            ldqt, colsum, ws, ws_bytes, stream);
}

extern "C" int df_quantize_2d_jit(int in_dtype, const void* x, int rows, int cols, int fmt, float* absmax_dev,
                                  float* scale_dev, uint8_t* q, int ldq, uint8_t* qt, int ldqt, float* colsum,
                                  void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    DF_CHECK(scale_dev, DF_ERR_INVALID, "df_quantize_2d_jit: scale_dev is NULL");
    return quantize_2d_impl("df_quantize_2d_jit", in_dtype, x, rows, cols, cols, fmt, scale_dev, q, ldq, qt, ldqt,
                            colsum, ws, ws_bytes, stream, nullptr, 0, nullptr, true, absmax_dev);
}

extern "C" int df_colsum(int in_dtype, const void* x, int rows, int cols, int ldx, float* out, void* ws,
                         size_t ws_bytes, void* stream) {
    // column sums alone: the same tile pass with no code outputs
    DF_CHECK(out, DF_ERR_INVALID, "df_colsum: out is NULL");
    return quantize_2d_impl("df_colsum", in_dtype, x, rows, cols, ldx, E4M3, nullptr, nullptr, 0, nullptr, 0, out,
                            ws, ws_bytes, stream);
}

extern "C" size_t df_quantize_2d_batch_workspace_bytes(void) { return kMaxReduceBlocks * sizeof(uint32_t); }

// absmax_in non-NULL: the per-tensor absmax comes from the caller (no
// absmax pass, no workspace); else it is measured into absmax_dev.
static int batch_impl(const char* name, int in_dtype, int count, const void* const* x, const int* rows,
                      const int* cols, int fmt, const float* absmax_in, float* absmax_dev, float* scale_dev,
                      uint8_t* const* q, const int* ldq, uint8_t* const* qt, const int* ldqt, void* ws,
                      size_t ws_bytes, void* stream) {
    clear_error();
    DF_CHECK(count >= 0, DF_ERR_INVALID, "%s: count=%d", name, count);
    if (count == 0) return DF_OK;
    DF_CHECK(x && rows && cols && scale_dev, DF_ERR_INVALID, "%s: NULL argument", name);
    DF_CHECK(fmt == E4M3 || fmt == E5M2, DF_ERR_UNSUPPORTED, "%s: bad format %d", name, fmt);
    DF_CHECK(in_dtype == DF_DTYPE_FLOAT32 || in_dtype == DF_DTYPE_BFLOAT16, DF_ERR_UNSUPPORTED,
             "%s: dtype %d not supported", name, in_dtype);
    DF_CHECK(aligned4(scale_dev) && aligned4(absmax_dev) && aligned4(absmax_in), DF_ERR_ALIGN,
             "%s: absmax/scale misaligned", name);
    DF_CHECK(absmax_in || (ws && aligned4(ws) && ws_bytes >= df_quantize_2d_batch_workspace_bytes()),
             DF_ERR_WORKSPACE, "%s: workspace %zu bytes < %zu", name, ws ? ws_bytes : (size_t)0,
             df_quantize_2d_batch_workspace_bytes());
    const int esz = in_dtype == DF_DTYPE_FLOAT32 ? 4 : 2;
    for (int t = 0; t < count; ++t) {
        uint8_t* qq = q ? q[t] : nullptr;
        uint8_t* qqt = qt ? qt[t] : nullptr;
        const bool empty = rows[t] == 0 || cols[t] == 0;
        DF_CHECK(rows[t] >= 0 && cols[t] >= 0, DF_ERR_INVALID, "%s: tensor %d: bad shape %d x %d", name, t, rows[t],
                 cols[t]);
        DF_CHECK(qq || qqt || empty, DF_ERR_INVALID, "%s: tensor %d: no output", name, t);
        DF_CHECK(x[t] || empty, DF_ERR_INVALID, "%s: tensor %d: x is NULL", name, t);
        DF_CHECK(aligned16(x[t]), DF_ERR_ALIGN, "%s: tensor %d: x must be 16-byte aligned", name, t);
        DF_CHECK(!qq || (ldq && ldq[t] >= cols[t] && ldq[t] % 16 == 0 && aligned16(qq)), DF_ERR_ALIGN,
                 "%s: tensor %d: q needs ldq >= cols, a multiple of 16, and 16-byte alignment", name, t);
        DF_CHECK(!qqt || (ldqt && ldqt[t] >= rows[t] && ldqt[t] % 16 == 0 && aligned16(qqt)), DF_ERR_ALIGN,
                 "%s: tensor %d: qt needs ldqt >= rows, a multiple of 16, and 16-byte alignment", name, t);
        DF_CHECK(q2d_grid(rows[t], cols[t], qq, qq ? ldq[t] : 0, qqt, qqt ? ldqt[t] : 0, kT2).y <= 65535, DF_ERR_INVALID,
                 "%s: tensor %d: rows=%d too large", name, t, rows[t]);
    }
    hipStream_t st = as_stream(stream);
    uint32_t* part = static_cast<uint32_t*>(ws);
    for (int t0 = 0; t0 < count; t0 += kBatchMax) {
        BatchArgs B{};
        B.count = std::min(count - t0, kBatchMax);
        // Each tensor's tile blocks form its scale themselves (no launch
        // between the passes) when every tensor has a tile to write it;
        // otherwise a separate fold or scale launch does.
        bool fold = true;
        for (int i = 0; i < B.count; ++i) fold = fold && rows[t0 + i] > 0 && cols[t0 + i] > 0;
        // absmax blocks in proportion to the tensors' sizes, at least one
        // each, at most kMaxReduceBlocks in all (kJitParts when every tile
        // block folds its tensor's partials)
        int64_t total = 0;
        for (int i = 0; i < B.count; ++i) total += (int64_t)rows[t0 + i] * cols[t0 + i];
        const int64_t budget = (fold ? kJitParts : kMaxReduceBlocks) - B.count;
        int bf = 0, tf = 0;
        for (int i = 0; i < B.count; ++i) {
            const int t = t0 + i;
            const int64_t n = (int64_t)rows[t] * cols[t];
            B.x[i] = x[t];
            B.rows[i] = rows[t];
            B.cols[i] = cols[t];
            B.q[i] = q ? q[t] : nullptr;
            B.qt[i] = qt ? qt[t] : nullptr;
            B.ldq[i] = B.q[i] ? ldq[t] : 0;
            B.ldqt[i] = B.qt[i] ? ldqt[t] : 0;
            B.vec_ok[i] = ((int64_t)cols[t] * esz) % 16 == 0;
            const int want = grid_for((n / (16 / esz) + kU - 1) / kU, kMaxReduceBlocks);
            const int share = total > 0 ? (int)((double)budget * (double)n / (double)total) : 0;
            B.blk_first[i] = bf;
            bf += 1 + std::max(0, std::min(want - 1, share));
            const dim3 g = q2d_grid(rows[t], cols[t], B.q[i], B.ldq[i], B.qt[i], B.ldqt[i], kT2);
            B.tile_first[i] = tf;
            B.tiles_x[i] = g.x > 0 ? (int)g.x : 1;
            tf += (int)(g.x * g.y);
        }
        B.blk_first[B.count] = bf;
        B.tile_first[B.count] = tf;
        float* am = absmax_dev ? absmax_dev + t0 : nullptr;
        float* sc = scale_dev + t0;
        if (!absmax_in) {
            if (in_dtype == DF_DTYPE_FLOAT32) absmax_batch_stage1<float><<<bf, kThreads, 0, st>>>(B, part);
            else absmax_batch_stage1<uint16_t><<<bf, kThreads, 0, st>>>(B, part);
            if (!fold) absmax_batch_stage2<<<B.count, kThreads, 0, st>>>(B, part, fmt, am, sc);
        } else if (!fold) {
            scale_batch_kernel<<<1, kThreads, 0, st>>>(absmax_in + t0, B.count, fmt, sc);
        }
        const float* ain = absmax_in ? absmax_in + t0 : nullptr;
        // non-temporal tiles where x is not in cache: no pass has just read it
        // (the caller's absmax), or the absmax pass read more than it holds
        auto tiles = [&](auto nt, auto src) {
            constexpr bool NT = decltype(nt)::value;
            constexpr int SRC = decltype(src)::value;
            if (in_dtype == DF_DTYPE_FLOAT32) {
                if (fmt == E4M3)
                    quantize_2d_batch_kernel<float, E4M3, NT, SRC><<<tf, kThreads, 0, st>>>(B, sc, part, ain, am, sc);
                else
                    quantize_2d_batch_kernel<float, E5M2, NT, SRC><<<tf, kThreads, 0, st>>>(B, sc, part, ain, am, sc);
            } else {
                if (fmt == E4M3)
                    quantize_2d_batch_kernel<uint16_t, E4M3, NT, SRC><<<tf, kThreads, 0, st>>>(B, sc, part, ain, am,
                                                                                            sc);
                else
                    quantize_2d_batch_kernel<uint16_t, E5M2, NT, SRC><<<tf, kThreads, 0, st>>>(B, sc, part, ain, am,
                                                                                            sc);
            }
        };
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        using S2 = std::integral_constant<int, 2>;
        if (tf > 0) {
            if (!fold) {
                if (absmax_in || total * esz > kBatchColdBytes) tiles(std::true_type(), S0());
                else tiles(std::false_type(), S0());
            } else if (absmax_in) {
                tiles(std::true_type(), S2());
            } else if (total * esz > kBatchColdBytes) {
                tiles(std::true_type(), S1());
            } else {
                tiles(std::false_type(), S1());
            }
        }
        if (int rc = launch_status(name)) return rc;
    }
    return DF_OK;
}

extern "C" int df_quantize_2d_batch(int in_dtype, int count, const void* const* x, const int* rows, const int* cols,
                                    int fmt, float* absmax_dev, float* scale_dev, uint8_t* const* q, const int* ldq,
                                    uint8_t* const* qt, const int* ldqt, void* ws, size_t ws_bytes, void* stream) {
    return batch_impl("df_quantize_2d_batch", in_dtype, count, x, rows, cols, fmt, nullptr, absmax_dev, scale_dev, q,
                      ldq, qt, ldqt, ws, ws_bytes, stream);
}

extern "C" int df_quantize_2d_batch_absmax(int in_dtype, int count, const void* const* x, const int* rows,
                                           const int* cols, int fmt, const float* absmax_dev, float* scale_dev,
                                           uint8_t* const* q, const int* ldq, uint8_t* const* qt, const int* ldqt,
                                           void* stream) {
    DF_CHECK(absmax_dev || count == 0, DF_ERR_INVALID, "df_quantize_2d_batch_absmax: absmax_dev is NULL");
    return batch_impl("df_quantize_2d_batch_absmax", in_dtype, count, x, rows, cols, fmt, absmax_dev, nullptr,
                      scale_dev, q, ldq, qt, ldqt, nullptr, 0, stream);
}

// ---------------------------------------------------------------- LayerNorm --
// Workspace: (mean, rstd) per row, then the absmax partials of the
// statistics pass or of the tile pass (delayed), 16-byte aligned.
static size_t ln_ws_layout(int rows, int cols, int ldq, int ldqt, size_t* part_off) {
    const size_t st = ((size_t)rows * sizeof(float2) + 15) & ~(size_t)15;
    const size_t stat_parts = (size_t)((rows + 3) / 4);
    const dim3 g = q2d_grid(rows, cols, (const uint8_t*)1, ldq, ldqt > 0 ? (const uint8_t*)1 : nullptr, ldqt, kT2R);
    const size_t tile_parts = (size_t)g.x * g.y;
    if (part_off) *part_off = st;
    return st + (stat_parts > tile_parts ? stat_parts : tile_parts) * sizeof(uint32_t) + 16;
}

extern "C" size_t df_layernorm_workspace_bytes(int rows, int cols, int ldq, int ldqt) {
    if (rows < 0 || cols < 0) return 0;
    return ln_ws_layout(rows, cols, ldq, ldqt, nullptr);
}

// mode 0: LayerNorm alone (y required); 1: just-in-time quantize (absmax of
// y in the statistics pass, scale written to *scale_dev before the tile
// pass reads it, the absmax itself to *next_scale when non-NULL); 2: delayed
// (scale_dev read, absmax in the tile pass, history pushed, next scale
// written)
static int layernorm_impl(const char* name, int mode, int dtype, const void* x, int rows, int cols, int ldx,
                          const void* gamma, const void* beta, float eps, void* y, int ldy, int fmt,
                          const float* scale_dev, float* next_scale, float* history, int len, uint8_t* q, int ldq,
                          uint8_t* qt, int ldqt, void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    DF_CHECK(rows >= 0 && cols >= 0 && (ldx >= cols || rows == 0), DF_ERR_INVALID,
             "%s: bad shape rows=%d cols=%d ldx=%d", name, rows, cols, ldx);
    DF_CHECK(dtype == DF_DTYPE_FLOAT32 || dtype == DF_DTYPE_BFLOAT16 || dtype == DF_DTYPE_HALF, DF_ERR_UNSUPPORTED,
             "%s: dtype %d not supported", name, dtype);
    DF_CHECK((gamma == nullptr) == (beta == nullptr), DF_ERR_INVALID, "%s: gamma and beta go together", name);
    DF_CHECK(eps >= 0.0f, DF_ERR_INVALID, "%s: eps < 0", name);
    const bool empty = rows == 0 || cols == 0;
    DF_CHECK(x || empty, DF_ERR_INVALID, "%s: x is NULL", name);
    if (mode == 0) DF_CHECK(y || empty, DF_ERR_INVALID, "%s: y is NULL", name);
    if (y) DF_CHECK(ldy >= cols, DF_ERR_INVALID, "%s: ldy=%d < cols", name, ldy);
    if (mode > 0) {
        DF_CHECK(fmt == E4M3 || fmt == E5M2, DF_ERR_UNSUPPORTED, "%s: bad format %d", name, fmt);
        DF_CHECK(scale_dev && aligned4(scale_dev), DF_ERR_INVALID, "%s: scale_dev NULL or misaligned", name);
        DF_CHECK(q || qt || empty, DF_ERR_INVALID, "%s: no code output", name);
        if (q) DF_CHECK(ldq >= cols && ldq % 16 == 0 && aligned16(q), DF_ERR_ALIGN, "%s: q layout (ldq=%d)", name, ldq);
        if (qt)
            DF_CHECK(ldqt >= rows && ldqt % 16 == 0 && aligned16(qt), DF_ERR_ALIGN, "%s: qt layout (ldqt=%d)", name,
                     ldqt);
    } else {
        q = qt = nullptr;
    }
    if (mode == 2) {
        DF_CHECK(history && next_scale && aligned4(history) && aligned4(next_scale), DF_ERR_INVALID,
                 "%s: history/next scale NULL or misaligned", name);
        DF_CHECK(len >= 1 && len <= kMaxHistory, DF_ERR_INVALID, "%s: history length %d not in [1, %d]", name, len,
                 kMaxHistory);
    }
    size_t part_off = 0;
    const size_t need = ln_ws_layout(rows, cols, q ? ldq : 0, qt ? ldqt : 0, &part_off);
    DF_CHECK(ws && aligned16(ws), DF_ERR_WORKSPACE, "%s: needs a 16-byte aligned workspace", name);
    DF_CHECK(ws_bytes >= need, DF_ERR_WORKSPACE, "%s: workspace %zu bytes < %zu", name, ws_bytes, need);
    hipStream_t st = as_stream(stream);
    float2* stat = static_cast<float2*>(ws);
    uint32_t* parts = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + part_off);
    const bool bf = dtype == DF_DTYPE_BFLOAT16, h16 = dtype == DF_DTYPE_HALF;
    // STMT once per element type, with T the kernels' element type
#define DF_BY_TYPE(STMT)            \
    do {                            \
        if (bf) {                   \
            using T = uint16_t;     \
            STMT;                   \
        } else if (h16) {           \
            using T = f16_t;        \
            STMT;                   \
        } else {                    \
            using T = float;        \
            STMT;                   \
        }                           \
    } while (0)
    if (empty) {
        // no values: absmax 0, scale 1 (stage 2 over no partials)
        if (mode == 1)
            absmax_stage2<<<1, kThreads, 0, st>>>(nullptr, 0, fmt, next_scale, const_cast<float*>(scale_dev));
        if (mode == 2) amax_history_kernel<<<1, kThreads, 0, st>>>(nullptr, 0, fmt, history, len, next_scale);
        return mode ? launch_status(name) : DF_OK;
    }
    // statistics pass
    const int sblocks = (rows + 3) / 4;
    const int esz = (bf || h16) ? 2 : 4;
    const bool vec_ok = aligned16(x) && ((int64_t)ldx * esz) % 16 == 0;
    const bool gb_vec = gamma && aligned16(gamma) && aligned16(beta);
#define DF_LNS(T, A)                                                                                           \
    ln_stats_kernel<T, A><<<sblocks, kThreads, 0, st>>>(static_cast<const T*>(x), rows, cols, ldx, vec_ok,     \
                                                        gb_vec, eps,                                            \
                                                        static_cast<const T*>(gamma), static_cast<const T*>(beta), \
                                                        stat, parts)
    DF_BY_TYPE(if (mode == 1) DF_LNS(T, true); else DF_LNS(T, false));
#undef DF_LNS
    if (mode == 1)
        absmax_stage2<<<1, kThreads, 0, st>>>(parts, sblocks, fmt, next_scale, const_cast<float*>(scale_dev));
    // tile pass
    LnArgs la;
    la.stat = stat;
    la.gamma = gamma;
    la.beta = beta;
    la.y = y;
    la.ldy = ldy;
    la.y_vec = y && aligned16(y) && ((int64_t)ldy * esz) % 16 == 0;
    const dim3 grid = q2d_grid(rows, cols, q, ldq, qt, ldqt, kT2R);
    DF_CHECK(grid.y <= 65535, DF_ERR_INVALID, "%s: rows=%d too large", name, rows);
#define DF_LNT(T, F, CODES, AMAX)                                                                              \
    quantize_2d_kernel<T, F, false, CODES, AMAX, true><<<grid, kThreads, 0, st>>>(                             \
        static_cast<const T*>(x), rows, cols, ldx, vec_ok, scale_dev, q, ldq, qt, ldqt, nullptr, parts, la)
    if (mode == 0) {
        DF_BY_TYPE(DF_LNT(T, E4M3, false, false));
    } else if (mode == 1) {
        DF_BY_TYPE(if (fmt == E4M3) DF_LNT(T, E4M3, true, false); else DF_LNT(T, E5M2, true, false));
    } else {
        DF_BY_TYPE(if (fmt == E4M3) DF_LNT(T, E4M3, true, true); else DF_LNT(T, E5M2, true, true));
        amax_history_kernel<<<1, kThreads, 0, st>>>(parts, (int)(grid.x * grid.y), fmt, history, len, next_scale);
    }
#undef DF_LNT
#undef DF_BY_TYPE
    return launch_status(name);
}

extern "C" int df_layernorm(int dtype, const void* x, int rows, int cols, int ldx, const void* gamma,
                            const void* beta, float eps, void* y, int ldy, void* ws, size_t ws_bytes, void* stream) {
    return layernorm_impl("df_layernorm", 0, dtype, x, rows, cols, ldx, gamma, beta, eps, y, ldy, E4M3, nullptr,
                          nullptr, nullptr, 0, nullptr, 0, nullptr, 0, ws, ws_bytes, stream);
}

extern "C" int df_layernorm_quantize(int dtype, const void* x, int rows, int cols, int ldx, const void* gamma,
                                     const void* beta, float eps, void* y, int ldy, int fmt, float* scale_dev,
                                     float* absmax_dev, uint8_t* q, int ldq, uint8_t* qt, int ldqt, void* ws,
                                     size_t ws_bytes, void* stream) {
    DF_CHECK(!absmax_dev || aligned4(absmax_dev), DF_ERR_ALIGN, "df_layernorm_quantize: absmax_dev misaligned");
    return layernorm_impl("df_layernorm_quantize", 1, dtype, x, rows, cols, ldx, gamma, beta, eps, y, ldy, fmt,
                          scale_dev, absmax_dev, nullptr, 0, q, ldq, qt, ldqt, ws, ws_bytes, stream);
}

extern "C" int df_layernorm_quantize_delayed(int dtype, const void* x, int rows, int cols, int ldx,
                                             const void* gamma, const void* beta, float eps, void* y, int ldy,
                                             int fmt, const float* scale_dev, float* next_scale_dev, float* history,
                                             int len, uint8_t* q, int ldq, uint8_t* qt, int ldqt, void* ws,
                                             size_t ws_bytes, void* stream) {
    return layernorm_impl("df_layernorm_quantize_delayed", 2, dtype, x, rows, cols, ldx, gamma, beta, eps, y, ldy,
                          fmt, scale_dev, next_scale_dev, history, len, q, ldq, qt, ldqt, ws, ws_bytes, stream);
}
