// gemm_fp8.hip -- fp8 "NT" GEMM on CDNA4 MFMA (gfx950):
//     C[m,n] = (sum_k A[m,k] * B[n,k]) * sa * sb + bias[n]
// A [M, lda] and B [N, ldb] are row-major fp8 with the reduction dimension
// contiguous, so both operands feed v_mfma_f32_16x16x128_f8f6f4 from LDS
// rows without a transpose.  The three Linear GEMMs are all this one shape:
//   forward  Y  = X  . W^T      A = X   [M, K]   B = W   [N, K]   (e4m3 x e4m3)
//   backward dX = dY . W        A = dY  [M, N]   B = W^T [K, N]   (e5m2 x e4m3)
//   backward dW = dY^T . X      A = dY^T[N, M]   B = X^T [K, M]   (e5m2 x e4m3)
// (the transposed operands come from df_quantize_2d's qt output).
//
// Tiling: a 256-thread block (4 waves, 2x2) owns a 128x128 tile of C; each
// wave owns 64x64 = 4x4 MFMA 16x16 tiles with fp32 accumulators.  K advances
// 128 bytes per step through two LDS buffers (global -> VGPR prefetch of the
// next step overlaps the MFMAs of the current one).  The epilogue applies
// the per-tensor scales and the bias and writes fp32 or bf16.
//
// Replaces the reference's fully_connected_forward_kernel, fc_backward_input
// and fc_backward_weights (dnn/layers/fully_connected_layer.cu:14-89).
#include <hip/hip_runtime.h>

#include "df_common.hpp"

namespace dfk {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBN = 128, kBK = 128;
constexpr int kLdsStride = kBK + 16;  // bytes per LDS row (pad breaks bank aliasing)
constexpr int kGemmThreads = 256;

template <typename T> struct OutCvt;
template <> struct OutCvt<float> {
    static __device__ __forceinline__ float cvt(float v) { return v; }
};
template <> struct OutCvt<uint16_t> {  // bf16 bits
    static __device__ __forceinline__ uint16_t cvt(float v) { return (uint16_t)f32_to_bf16_rne(v); }
};
__device__ __forceinline__ float bias_ld(const float* b, int i) { return b[i]; }
__device__ __forceinline__ float bias_ld(const uint16_t* b, int i) { return bf16_to_f32(b[i]); }

__device__ __forceinline__ v8i lds_frag(const uint8_t* p) {
    const uint4 lo = *reinterpret_cast<const uint4*>(p);
    const uint4 hi = *reinterpret_cast<const uint4*>(p + 16);
    v8i r;
    r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
    r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
    return r;
}

template <int FA, int FB, typename OutT, typename BiasT>
__global__ __launch_bounds__(kGemmThreads, 2) void gemm_nt_kernel(
    const uint8_t* __restrict__ A, int lda, const uint8_t* __restrict__ B, int ldb, int M, int N,
    int K, const float* __restrict__ sa, const float* __restrict__ sb,
    const BiasT* __restrict__ bias, OutT* __restrict__ C, int ldc) {
    __shared__ __attribute__((aligned(16))) uint8_t sA[2][kBM * kLdsStride];
    __shared__ __attribute__((aligned(16))) uint8_t sB[2][kBN * kLdsStride];

    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int wm = w >> 1, wn = w & 1;
    const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;

    // global -> register staging: thread t moves 16-byte chunks of rows
    // t/8 + 32*i, column (t%8)*16 of each operand tile.
    const int lrow = t >> 3, lcol = (t & 7) * 16;
    uint4 ra[4], rb[4];
    auto gload = [&](int k0) {
        const int gk = k0 + lcol;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = lrow + 32 * i;
            const int gm = m0 + r, gn = n0 + r;
            ra[i] = (gm < M && gk < K) ? *reinterpret_cast<const uint4*>(A + (int64_t)gm * lda + gk)
                                       : make_uint4(0, 0, 0, 0);
            rb[i] = (gn < N && gk < K) ? *reinterpret_cast<const uint4*>(B + (int64_t)gn * ldb + gk)
                                       : make_uint4(0, 0, 0, 0);
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = lrow + 32 * i;
            *reinterpret_cast<uint4*>(&sA[buf][r * kLdsStride + lcol]) = ra[i];
            *reinterpret_cast<uint4*>(&sB[buf][r * kLdsStride + lcol]) = rb[i];
        }
    };

    v4f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    const int nk = (K + kBK - 1) / kBK;
    gload(0);
    lstore(0);
    __syncthreads();

    // MFMA operand layout (16x16x128, 8-bit): lane l supplies row l%16 of
    // its operand and 32 bytes of K at byte offset 32*(l/16); A and B share
    // the layout, so both read their own rows the same way.
    const int fr = lane & 15, fk = (lane >> 4) * 32;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * kBK);
        v8i af[4], bf[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            af[i] = lds_frag(&sA[cur][(wm * 64 + i * 16 + fr) * kLdsStride + fk]);
            bf[i] = lds_frag(&sB[cur][(wn * 64 + i * 16 + fr) * kLdsStride + fk]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[i], bf[j], acc[i][j], FA,
                                                                             FB, 0, 0, 0, 0);
        if (kt + 1 < nk) lstore(cur ^ 1);
        __syncthreads();
    }

    // Epilogue.  Accumulator layout (16x16 fp32): lane l holds column l%16,
    // rows 4*(l/16) + r for r = 0..3.
    const float sab = sa[0] * sb[0];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = n0 + wn * 64 + j * 16 + (lane & 15);
            if (col >= N) continue;
            const float bv = bias ? bias_ld(bias, col) : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
                if (row < M) C[(int64_t)row * ldc + col] = OutCvt<OutT>::cvt(acc[i][j][r] * sab + bv);
            }
        }
}

template <int FA, int FB, typename OutT, typename BiasT>
static void launch_gemm(const uint8_t* A, int lda, const uint8_t* B, int ldb, int M, int N, int K,
                        const float* sa, const float* sb, const void* bias, void* C, int ldc,
                        hipStream_t st) {
    dim3 grid((N + kBN - 1) / kBN, (M + kBM - 1) / kBM);
    gemm_nt_kernel<FA, FB, OutT, BiasT><<<grid, kGemmThreads, 0, st>>>(
        A, lda, B, ldb, M, N, K, sa, sb, static_cast<const BiasT*>(bias), static_cast<OutT*>(C), ldc);
}

template <int FA, int FB>
static int dispatch_out(const uint8_t* A, int lda, const uint8_t* B, int ldb, int M, int N, int K,
                        const float* sa, const float* sb, int bias_dtype, const void* bias,
                        int c_dtype, void* C, int ldc, hipStream_t st) {
    const bool bf16_bias = bias && bias_dtype == DF_DTYPE_BFLOAT16;
    if (c_dtype == DF_DTYPE_FLOAT32) {
        if (bf16_bias) launch_gemm<FA, FB, float, uint16_t>(A, lda, B, ldb, M, N, K, sa, sb, bias, C, ldc, st);
        else launch_gemm<FA, FB, float, float>(A, lda, B, ldb, M, N, K, sa, sb, bias, C, ldc, st);
    } else {
        if (bf16_bias) launch_gemm<FA, FB, uint16_t, uint16_t>(A, lda, B, ldb, M, N, K, sa, sb, bias, C, ldc, st);
        else launch_gemm<FA, FB, uint16_t, float>(A, lda, B, ldb, M, N, K, sa, sb, bias, C, ldc, st);
    }
    return DF_OK;
}

}  // namespace dfk

using namespace dfk;

extern "C" int df_fp8_gemm_nt(int fmt_a, const uint8_t* A, int lda, int fmt_b, const uint8_t* B,
                              int ldb, int M, int N, int K, const float* scale_a_dev,
                              const float* scale_b_dev, int bias_dtype, const void* bias,
                              int c_dtype, void* C, int ldc, void* stream) {
    clear_error();
    DF_CHECK(M >= 0 && N >= 0 && K >= 0, DF_ERR_INVALID, "df_fp8_gemm_nt: negative size M=%d N=%d K=%d", M, N, K);
    DF_CHECK((fmt_a == E4M3 || fmt_a == E5M2) && (fmt_b == E4M3 || fmt_b == E5M2), DF_ERR_UNSUPPORTED,
             "df_fp8_gemm_nt: bad fp8 formats %d %d", fmt_a, fmt_b);
    DF_CHECK(c_dtype == DF_DTYPE_FLOAT32 || c_dtype == DF_DTYPE_BFLOAT16, DF_ERR_UNSUPPORTED,
             "df_fp8_gemm_nt: output dtype %d not supported", c_dtype);
    DF_CHECK(!bias || bias_dtype == DF_DTYPE_FLOAT32 || bias_dtype == DF_DTYPE_BFLOAT16, DF_ERR_UNSUPPORTED,
             "df_fp8_gemm_nt: bias dtype %d not supported", bias_dtype);
    DF_CHECK(ldc >= N, DF_ERR_INVALID, "df_fp8_gemm_nt: ldc=%d < N=%d", ldc, N);
    if (M == 0 || N == 0) return DF_OK;
    DF_CHECK(A && B && C && scale_a_dev && scale_b_dev, DF_ERR_INVALID, "df_fp8_gemm_nt: NULL pointer");
    DF_CHECK(lda >= K && ldb >= K && lda % 16 == 0 && ldb % 16 == 0, DF_ERR_ALIGN,
             "df_fp8_gemm_nt: lda=%d ldb=%d must be multiples of 16 and >= K=%d", lda, ldb, K);
    DF_CHECK(aligned16(A) && aligned16(B), DF_ERR_ALIGN, "df_fp8_gemm_nt: A and B must be 16-byte aligned");
    DF_CHECK((M + kBM - 1) / kBM <= 65535, DF_ERR_INVALID, "df_fp8_gemm_nt: M=%d too large", M);
    // K is rounded up to the 16-byte granule: the operand rows are zero
    // there (df_quantize_2d pads ld with zeros), so the products vanish.
    const int Kp = (K + 15) & ~15;
    hipStream_t st = as_stream(stream);
    if (fmt_a == E4M3 && fmt_b == E4M3)
        dispatch_out<E4M3, E4M3>(A, lda, B, ldb, M, N, Kp, scale_a_dev, scale_b_dev, bias_dtype, bias, c_dtype, C, ldc, st);
    else if (fmt_a == E5M2 && fmt_b == E4M3)
        dispatch_out<E5M2, E4M3>(A, lda, B, ldb, M, N, Kp, scale_a_dev, scale_b_dev, bias_dtype, bias, c_dtype, C, ldc, st);
    else if (fmt_a == E4M3 && fmt_b == E5M2)
        dispatch_out<E4M3, E5M2>(A, lda, B, ldb, M, N, Kp, scale_a_dev, scale_b_dev, bias_dtype, bias, c_dtype, C, ldc, st);
    else
        dispatch_out<E5M2, E5M2>(A, lda, B, ldb, M, N, Kp, scale_a_dev, scale_b_dev, bias_dtype, bias, c_dtype, C, ldc, st);
    return launch_status("df_fp8_gemm_nt");
}

extern "C" int df_fp8_gemm_fwd(const uint8_t* Xq, int ldx, const uint8_t* Wq, int ldw, int M, int N,
                               int K, const float* sx_dev, const float* sw_dev, int bias_dtype,
                               const void* bias, int y_dtype, void* Y, int ldy, void* stream) {
    return df_fp8_gemm_nt(DF_FMT_E4M3, Xq, ldx, DF_FMT_E4M3, Wq, ldw, M, N, K, sx_dev, sw_dev,
                          bias_dtype, bias, y_dtype, Y, ldy, stream);
}

extern "C" int df_fp8_gemm_bwd_dx(const uint8_t* dYq, int lddy, const uint8_t* Wtq, int ldwt, int M,
                                  int N, int K, const float* sdy_dev, const float* sw_dev,
                                  int dx_dtype, void* dX, int lddx, void* stream) {
    // dX[M,K] = sum_n dY[m,n] W[n,k]: NT with reduction N, B = W^T [K, N]
    return df_fp8_gemm_nt(DF_FMT_E5M2, dYq, lddy, DF_FMT_E4M3, Wtq, ldwt, M, K, N, sdy_dev, sw_dev,
                          DF_DTYPE_FLOAT32, nullptr, dx_dtype, dX, lddx, stream);
}

extern "C" int df_fp8_gemm_bwd_dw(const uint8_t* dYtq, int ldyt, const uint8_t* Xtq, int ldxt, int M,
                                  int N, int K, const float* sdy_dev, const float* sx_dev,
                                  int dw_dtype, void* dW, int lddw, void* stream) {
    // dW[N,K] = sum_m dY[m,n] X[m,k]: NT with reduction M, A = dY^T [N, M], B = X^T [K, M]
    return df_fp8_gemm_nt(DF_FMT_E5M2, dYtq, ldyt, DF_FMT_E4M3, Xtq, ldxt, N, K, M, sdy_dev, sx_dev,
                          DF_DTYPE_FLOAT32, nullptr, dw_dtype, dW, lddw, stream);
}
