/*
 * df_capi.h -- C ABI of the MI355X-native fp8 Linear path (libdeepfuse_amd.so).
 *
 * The reference (SensorVista/DeepFuse) has no C ABI: its host code calls
 * CUDA kernels directly from C++ (dnn/layers/fully_connected_layer.cu:164-357,
 * dnn/core/tensor.cu:77-462).  Each entry point below names the reference
 * function or kernel it replaces.  The C++ drop-in API (deepfuse_amd/dnn/...,
 * namespace dnn) calls only these entry points for device work.
 *
 * Conventions
 *  - Pointers named *_dev, x, q, out, A, B, C, ws are DEVICE pointers.
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *    Every call only enqueues work; nothing synchronises the host.
 *  - Return value: DF_OK (0) or a negative df_status.  Nothing throws across
 *    the ABI.  df_last_error_string() gives the calling thread's last message.
 *  - Element counts are int64_t; matrix dimensions are int (the reference's
 *    tensor uses int shapes, dnn/core/tensor.cuh:26-28).
 *  - Calls on different streams are independent and thread-safe; a workspace
 *    or output buffer must not be shared by calls that may overlap.
 *  - Per-tensor scale (contract D1/D2): s = absmax / FMAX with FMAX = 448
 *    (e4m3) or 57344 (e5m2); absmax is over finite values; absmax == 0 gives
 *    s = 1.  Quantize: q = sat_rne(x / s) (IEEE binary32 division, then
 *    round-to-nearest-even into OCP fp8, saturating; NaN -> sign|0x7F,
 *    +-inf -> +-max).  Dequantize: decode(q) * s in binary32; bf16 output is
 *    the RNE rounding of that binary32; NaN codes give the canonical quiet NaN.
 */
#ifndef DF_CAPI_H
#define DF_CAPI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
typedef enum {
    DF_OK = 0,
    DF_ERR_INVALID = -1,     /* null pointer, negative or inconsistent size */
    DF_ERR_UNSUPPORTED = -2, /* dtype / format combination not provided */
    DF_ERR_HIP = -3,         /* HIP runtime reported an error */
    DF_ERR_ALIGN = -4,       /* pointer or leading dimension misaligned */
    DF_ERR_WORKSPACE = -5    /* workspace too small */
} df_status;

/* ---- fp8 formats (OCP OFP8 v1.0) ---- */
typedef enum { DF_FMT_E4M3 = 0, DF_FMT_E5M2 = 1 } df_fp8_format;

/* ---- element types: values 0-4 are the reference's own enum
 * OnnxLoader::DType (dnn/utils/onnx_loader.cuh:16-22); 5 and 6 extend it
 * with the two 1-byte fp8 formats; 7 is int32 (the reference's tensor<int>,
 * dnn/core/tensor.cu:486). ---- */
typedef enum {
    DF_DTYPE_FLOAT32 = 0,
    DF_DTYPE_HALF = 1,
    DF_DTYPE_INT8 = 2,
    DF_DTYPE_UINT8 = 3,
    DF_DTYPE_BFLOAT16 = 4,
    DF_DTYPE_FP8E4M3 = 5,
    DF_DTYPE_FP8E5M2 = 6,
    DF_DTYPE_INT32 = 7
} df_dtype;

/* ---- library ---- */
const char* df_last_error_string(void);   /* thread-local, never NULL */
int df_version(void);                     /* 100 * major + minor */
int df_device_arch_ok(void);              /* 1 when the current device is gfx950 */

/* ---- absmax / scale (new: the reference has no quantizer, README.md:16) ----
 * Two-stage reduction: a grid pass writes per-block maxima into `ws`, a
 * single-block pass folds them and writes absmax and the scale.  `ws` must
 * hold df_absmax_workspace_bytes() bytes. */
size_t df_absmax_workspace_bytes(void);
int df_absmax_f32(const float* x, int64_t n, float* absmax_dev,
                  void* ws, size_t ws_bytes, void* stream);
int df_absmax_bf16(const uint16_t* x, int64_t n, float* absmax_dev,
                   void* ws, size_t ws_bytes, void* stream);
/* x: binary16 bits (DF_DTYPE_HALF) */
int df_absmax_f16(const uint16_t* x, int64_t n, float* absmax_dev,
                  void* ws, size_t ws_bytes, void* stream);
/* absmax and the scale for `fmt` in one call (scale_dev may equal NULL). */
int df_absmax_scale_f32(const float* x, int64_t n, int fmt, float* absmax_dev,
                        float* scale_dev, void* ws, size_t ws_bytes, void* stream);
int df_absmax_scale_bf16(const uint16_t* x, int64_t n, int fmt, float* absmax_dev,
                         float* scale_dev, void* ws, size_t ws_bytes, void* stream);
int df_absmax_scale_f16(const uint16_t* x, int64_t n, int fmt, float* absmax_dev,
                        float* scale_dev, void* ws, size_t ws_bytes, void* stream);
/* ---- bandwidth calibration (measurement only; no reference counterpart)
 * The flat absmax / quantize / dequantize kernels' exact access pattern
 * without their arithmetic, to measure the HBM ceiling each conversion can
 * reach on this part: src_bytes of src read as read_bytes per vector (16
 * bytes per lane-load, 8 loads in flight per thread, non-temporal) and, per
 * vector, write_bytes stored to dst (an XOR fold of the loaded words).
 * Patterns (read:write bytes) 16:0 (absmax; dst gets one word per block),
 * 16:4 (fp32 -> fp8), 16:8 (bf16 -> fp8), 4:16 (fp8 -> fp32), 8:16 (fp8 ->
 * bf16), 16:16 (a copy).  src_bytes must be a multiple of 2048 * read_bytes;
 * dst holds df_hbm_probe_dst_bytes(...) bytes. */
size_t df_hbm_probe_dst_bytes(int read_bytes, int write_bytes, int64_t src_bytes);
int df_hbm_probe(int read_bytes, int write_bytes, const void* src, int64_t src_bytes, void* dst,
                 void* stream);

/* scale from an absmax already on the device */
int df_compute_scale(const float* absmax_dev, int fmt, float* scale_dev, void* stream);

/* ---- quantize (new; element type of the reference's fp8 instantiations,
 * dnn/core/tensor.cu:489-498, made 1 byte per value) ----
 * x and q must be 16-byte aligned for the vector path; any n >= 0. */
int df_quantize_f32_e4m3(const float* x, int64_t n, const float* scale_dev,
                         uint8_t* q, void* stream);
int df_quantize_f32_e5m2(const float* x, int64_t n, const float* scale_dev,
                         uint8_t* q, void* stream);
int df_quantize_bf16_e4m3(const uint16_t* x, int64_t n, const float* scale_dev,
                          uint8_t* q, void* stream);
int df_quantize_bf16_e5m2(const uint16_t* x, int64_t n, const float* scale_dev,
                          uint8_t* q, void* stream);

/* ---- dequantize (new) ---- */
int df_dequantize_e4m3_f32(const uint8_t* q, int64_t n, const float* scale_dev,
                           float* out, void* stream);
int df_dequantize_e5m2_f32(const uint8_t* q, int64_t n, const float* scale_dev,
                           float* out, void* stream);
int df_dequantize_e4m3_bf16(const uint8_t* q, int64_t n, const float* scale_dev,
                            uint16_t* out, void* stream);
int df_dequantize_e5m2_bf16(const uint8_t* q, int64_t n, const float* scale_dev,
                            uint16_t* out, void* stream);

/* ---- 2-D quantize into GEMM operand layout (new) ----
 * x: row-major [rows, cols] with leading dimension ldx (elements), dtype
 * DF_DTYPE_FLOAT32, DF_DTYPE_HALF or DF_DTYPE_BFLOAT16 (both 2-byte types
 * widen to binary32 exactly before the code is taken).  Writes, when non-NULL:
 *   q  [rows, ldq]  : q[r*ldq + c] = code(x[r,c]); columns [cols, ldq) = 0
 *   qt [cols, ldqt] : qt[c*ldqt + r] = code(x[r,c]); columns [rows, ldqt) = 0
 * ldq and ldqt must be multiples of 16 (the GEMM's K granule).  qt is the
 * transposed copy the backward GEMMs read (dX needs W^T, dW needs dY^T and
 * X^T), produced in the same pass as q. */
int df_quantize_2d(int in_dtype, const void* x, int rows, int cols, int ldx,
                   int fmt, const float* scale_dev, uint8_t* q, int ldq,
                   uint8_t* qt, int ldqt, void* stream);
/* Workspace for the column-sum passes below: ceil(rows/128) * cols floats. */
size_t df_quantize_2d_workspace_bytes(int rows, int cols);
/* df_quantize_2d plus colsum[c] = sum_r x[r,c] in fp32 from the same read of
 * x (the bias gradient of the upstream gradient dY, replacing
 * fc_backward_bias, dnn/layers/fully_connected_layer.cu:91-106).  Sums run
 * over each 128-row tile, then over tiles in order: deterministic, but not
 * the reference's sequential order.  q and qt may both be NULL. */
int df_quantize_2d_colsum(int in_dtype, const void* x, int rows, int cols, int ldx,
                          int fmt, const float* scale_dev, uint8_t* q, int ldq,
                          uint8_t* qt, int ldqt, float* colsum,
                          void* ws, size_t ws_bytes, void* stream);
/* Just-in-time quantize in one call (new; the reference has no quantizer,
 * README.md:16): df_absmax_scale_* of x, then df_quantize_2d (colsum NULL)
 * or df_quantize_2d_colsum at that scale, with the same absmax, scale, codes
 * and column sums, bit for bit.  *scale_dev (required) and *absmax_dev (may
 * be NULL) are outputs.  x is contiguous [rows, cols] and 16-byte aligned.
 * The tile pass forms the scale from the absmax partials itself, so no
 * one-block launch sits between the two passes.  ws:
 * df_quantize_2d_jit_workspace_bytes(rows, cols, colsum != NULL). */
size_t df_quantize_2d_jit_workspace_bytes(int rows, int cols, int colsum);
int df_quantize_2d_jit(int in_dtype, const void* x, int rows, int cols, int fmt,
                       float* absmax_dev, float* scale_dev, uint8_t* q, int ldq,
                       uint8_t* qt, int ldqt, float* colsum,
                       void* ws, size_t ws_bytes, void* stream);

/* ---- column sums alone (replaces fc_backward_bias,
 * dnn/layers/fully_connected_layer.cu:91-106) ----
 * out[c] = sum_r x[r, c] in fp32, same order as df_quantize_2d_colsum;
 * overwrites out.  ws: df_quantize_2d_workspace_bytes(rows, cols) bytes. */
int df_colsum(int in_dtype, const void* x, int rows, int cols, int ldx,
              float* out, void* ws, size_t ws_bytes, void* stream);

/* Several contiguous 2-D tensors x[t] [rows[t], cols[t]] (every Linear's
 * weights after an optimizer step) in two launches (three when a tensor is
 * empty) instead of three per tensor: per-tensor absmax and scale into
 * absmax_dev[t] (device array, or
 * NULL) and scale_dev[t] (device array), then row codes q[t] [rows, ldq[t]]
 * and transposed codes qt[t] [cols, ldqt[t]] (either pointer array, or any
 * entry, may be NULL), zero-padded like df_quantize_2d.  Each tensor gets
 * exactly the scale and codes df_absmax_scale_* followed by df_quantize_2d
 * gives it.  x, rows, cols, q, ldq, qt and ldqt are HOST arrays of `count`
 * entries holding device pointers and sizes; x[t] 16-byte aligned.  ws:
 * df_quantize_2d_batch_workspace_bytes() bytes.  No reference counterpart:
 * the reference quantizes nothing; per tensor this is a5 + a6. */
size_t df_quantize_2d_batch_workspace_bytes(void);
int df_quantize_2d_batch(int in_dtype, int count, const void* const* x, const int* rows,
                         const int* cols, int fmt, float* absmax_dev, float* scale_dev,
                         uint8_t* const* q, const int* ldq, uint8_t* const* qt,
                         const int* ldqt, void* ws, size_t ws_bytes, void* stream);
/* The same with the per-tensor absmax given (absmax_dev[t], device array),
 * e.g. from df_adam_update_absmax_f32: no absmax pass, no workspace; the
 * scales are formed from it by the D1/D2 rule, as df_compute_scale does. */
int df_quantize_2d_batch_absmax(int in_dtype, int count, const void* const* x, const int* rows,
                                const int* cols, int fmt, const float* absmax_dev, float* scale_dev,
                                uint8_t* const* q, const int* ldq, uint8_t* const* qt,
                                const int* ldqt, void* stream);

/* ---- delayed scaling (new: the reference has no quantizer) ----
 * The scale of a tensor comes from an amax history of earlier passes instead
 * of an absmax pass over the current data.  history[0..len) (device, fp32,
 * len <= 1024, history[0] newest) and scale_dev belong to one tensor role
 * (e.g. one layer's X, W or dY).
 *  df_amax_history_init    : history[i] = *amax_dev (0 when amax_dev is
 *                            NULL or *amax_dev is not a positive finite
 *                            value), *scale_dev = scale rule D1/D2 of it.
 *  df_quantize_2d_delayed  : df_quantize_2d / df_quantize_2d_colsum at
 *                            the scale *scale_dev (codes saturate beyond
 *                            FMAX * scale, D3); the same pass measures the
 *                            input's absmax (finite values), pushes it to
 *                            history[0] (older entries move up one, the
 *                            oldest drops out) and then writes the scale of
 *                            the maximum over the new history to
 *                            *next_scale_dev, for the next call.
 *                            next_scale_dev may equal scale_dev when the
 *                            caller no longer needs the scale of these codes
 *                            (the GEMMs that read it are enqueued before the
 *                            next call otherwise).  colsum may be NULL.  ws
 *                            holds df_quantize_2d_delayed_workspace_bytes(
 *                            rows, cols, ldq or 0, ldqt or 0,
 *                            colsum != NULL) bytes, 16-byte aligned. */
int df_amax_history_init(const float* amax_dev, int fmt, float* history, int len, float* scale_dev,
                         void* stream);
size_t df_quantize_2d_delayed_workspace_bytes(int rows, int cols, int ldq, int ldqt, int colsum);
int df_quantize_2d_delayed(int in_dtype, const void* x, int rows, int cols, int ldx, int fmt,
                           const float* scale_dev, float* next_scale_dev, float* history, int len,
                           uint8_t* q, int ldq, uint8_t* qt, int ldqt, float* colsum, void* ws,
                           size_t ws_bytes, void* stream);

/* df_quantize_2d_delayed without a workspace argument: the allocation-free
 * variant, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference (which quantizes nothing).  Its workspace is
 * a fixed array of DF_QUANTIZE_2D_NOALLOC_SCRATCH_BYTES inside the library,
 * one per GPU, held until the process ends; the call allocates nothing
 * (no hipMalloc, hipFree or allocating library routine).  A shape whose
 * workspace (df_quantize_2d_delayed_workspace_bytes) exceeds that size is
 * refused with DF_ERR_WORKSPACE before anything is launched.  Results are
 * bit-identical to df_quantize_2d_delayed's.  Every call on one GPU uses
 * that GPU's one array: calls that may overlap on one GPU (different
 * streams, different threads) race and must be serialised by the caller. */
#define DF_QUANTIZE_2D_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int df_quantize_2d_delayed_noalloc(int in_dtype, const void* x, int rows, int cols, int ldx, int fmt,
                                   const float* scale_dev, float* next_scale_dev, float* history,
                                   int len, uint8_t* q, int ldq, uint8_t* qt, int ldqt,
                                   float* colsum, void* stream);

/* ---- LayerNorm with the quantize of its output fused in (producer side of
 * the qkv / fc1 Linears; layer_norm_forward_kernel,
 * dnn/layers/layer_norm_layer.cu:26-63) ----
 * Per row of x [rows, cols] (ldx elements apart), dtype fp32, f16 or bf16:
 *   mean = sum(x)/cols, var = sum((x - mean)^2)/cols, rstd = 1/sqrt(var + eps)
 *   y = (x - mean) * rstd, then y = fma(y, gamma, beta) when gamma/beta
 *   (both [cols], same dtype) are given; y is rounded to the dtype (RNE).
 * Sums are binary32, per-lane strided then a fixed butterfly: deterministic,
 * not the reference's sequential order.
 *  df_layernorm                 : writes y [rows, ldy].
 *  df_layernorm_quantize        : codes of y at the just-in-time scale
 *                                 (*scale_dev = D1/D2 of absmax(y), measured
 *                                 in the statistics pass; *absmax_dev =
 *                                 absmax(y) when non-NULL), q [rows, ldq]
 *                                 and/or qt [cols, ldqt] as df_quantize_2d
 *                                 writes them; y [rows, ldy] too when
 *                                 non-NULL.  The codes equal
 *                                 df_quantize_2d of df_layernorm's y.
 *  df_layernorm_quantize_delayed: the same at *scale_dev from an amax
 *                                 history (see df_quantize_2d_delayed).
 * x is read twice (statistics, then the tile pass) and y need not be
 * written at all.  ws: df_layernorm_workspace_bytes(rows, cols, ldq or 0,
 * ldqt or 0) bytes, 16-byte aligned. */
size_t df_layernorm_workspace_bytes(int rows, int cols, int ldq, int ldqt);
int df_layernorm(int dtype, const void* x, int rows, int cols, int ldx, const void* gamma,
                 const void* beta, float eps, void* y, int ldy, void* ws, size_t ws_bytes,
                 void* stream);
int df_layernorm_quantize(int dtype, const void* x, int rows, int cols, int ldx,
                          const void* gamma, const void* beta, float eps, void* y, int ldy,
                          int fmt, float* scale_dev, float* absmax_dev, uint8_t* q, int ldq,
                          uint8_t* qt, int ldqt, void* ws, size_t ws_bytes, void* stream);
int df_layernorm_quantize_delayed(int dtype, const void* x, int rows, int cols, int ldx,
                                  const void* gamma, const void* beta, float eps, void* y,
                                  int ldy, int fmt, const float* scale_dev,
                                  float* next_scale_dev, float* history, int len, uint8_t* q,
                                  int ldq, uint8_t* qt, int ldqt, void* ws, size_t ws_bytes,
                                  void* stream);

/* ---- fp8 GEMM, "NT": C[m,n] = (sum_k A[m,k] * B[n,k]) * sa * sb + bias[n]
 *   A [M, lda] fp8 (fmt_a), B [N, ldb] fp8 (fmt_b), both row-major with the
 *   reduction dimension contiguous; lda, ldb multiples of 16 and >= K;
 *   A, B 16-byte aligned; sa, sb device scalars; bias NULL or [N] of
 *   bias_dtype; C [M, ldc] of c_dtype, overwritten: an FLOAT32 or BFLOAT16
 *   C with an FLOAT32 or BFLOAT16 bias, or a HALF C (the FP16 layer's) with
 *   an FLOAT32 or HALF bias; a 2-byte C is rounded to nearest even.  fp32
 *   accumulation on CDNA4 fp8 MFMA.
 *   When K is not a multiple of 16, columns [K, roundup(K,16)) of A and B
 *   must hold zero codes (df_quantize_2d writes its padding that way).
 *   ws / ws_bytes: optional device workspace (16-byte aligned) for split-K
 *   partial tiles on outputs too small to fill the GPU; NULL or too small
 *   only turns split-K off.  df_fp8_gemm_workspace_bytes() is the size that
 *   never limits it.  Results do not depend on run-to-run timing (split-K
 *   partials are summed in a fixed order).
 * Replaces fully_connected_forward_kernel (fully_connected_layer.cu:14-41). */
size_t df_fp8_gemm_workspace_bytes(int M, int N, int K);
int df_fp8_gemm_nt(int fmt_a, const uint8_t* A, int lda,
                   int fmt_b, const uint8_t* B, int ldb,
                   int M, int N, int K,
                   const float* scale_a_dev, const float* scale_b_dev,
                   int bias_dtype, const void* bias,
                   int c_dtype, void* C, int ldc,
                   void* ws, size_t ws_bytes, void* stream);

/* The kernel df_fp8_gemm_nt runs for these arguments (bias: the bias
 * pointer the call would pass, or NULL -- only its alignment matters;
 * ws_bytes: the workspace size, 0 for none): *kernel one of
 * DF_GEMM_KERNEL_*, *split the K slices (1 = unsplit).  The persistent
 * kernel takes every call whose operands fit its 32-bit buffer offsets
 * (M*lda and N*ldb below 2^31, lda and ldb below 2^23) and whose bias is
 * 4-byte aligned, with 256x256 tiles or, where its rounds cost model
 * prefers them, 256x128 tiles (PERSISTENT_NARROW); the tiled kernels take
 * the rest, with LDS-DMA operand
 * loads while M*lda and N*ldb stay below 2^31 and register-staged loads
 * beyond.  Same plan as the reference-facing calls below; no reference
 * counterpart (the reference has one kernel per GEMM). */
enum {
    DF_GEMM_KERNEL_PERSISTENT = 0,
    DF_GEMM_KERNEL_TILED_DMA_256 = 1,
    DF_GEMM_KERNEL_TILED_DMA_128 = 2,
    DF_GEMM_KERNEL_TILED_REG_256 = 3,
    DF_GEMM_KERNEL_TILED_REG_128 = 4,
    DF_GEMM_KERNEL_PERSISTENT_NARROW = 5
};
int df_fp8_gemm_nt_plan(int M, int N, int K, int lda, int ldb, const void* bias, size_t ws_bytes,
                        int* kernel, int* split);

/* Forward: Y[M,N] = X_q[M,K] . W_q[N,K]^T * sx * sw + b  (e4m3 x e4m3).
 * Replaces fully_connected_forward_kernel (fully_connected_layer.cu:14-41). */
int df_fp8_gemm_fwd(const uint8_t* Xq, int ldx, const uint8_t* Wq, int ldw,
                    int M, int N, int K, const float* sx_dev, const float* sw_dev,
                    int bias_dtype, const void* bias, int y_dtype, void* Y, int ldy,
                    void* ws, size_t ws_bytes, void* stream);
/* The forward above on its unsplit 256x256 persistent kernel, bf16 bias
 * and bf16 Y only, with a per-tile timeline (diagnostic; no counterpart in
 * the reference): stamps[b * stamps_per_block + i] gets the GPU's 100 MHz
 * real-time counter for block b at its start (i = 0) and, for its t-th
 * tile, at the tile's first half-step (1 + 3t), before its epilogue
 * (2 + 3t) and after it (3 + 3t), as far as stamps_per_block reaches;
 * *grid_out = the blocks launched.  Y is the forward's Y.  Shapes whose plan
 * is not that kernel are DF_ERR_UNSUPPORTED. */
int df_fp8_gemm_fwd_timeline(const uint8_t* Xq, int ldx, const uint8_t* Wq, int ldw, int M, int N, int K,
                             const float* sx_dev, const float* sw_dev, const uint16_t* bias_bf16,
                             uint16_t* Y_bf16, int ldy, uint64_t* stamps, int stamps_per_block,
                             int* grid_out, void* stream);
/* The forward GEMM of df_fp8_gemm_fwd whose Y also gives the absmax the next
 * Linear's just-in-time scale needs (new; no counterpart in the reference,
 * whose TransformerBlock feeds fc1's output straight into fc2,
 * dnn/layers/transformer_block.cu:79-81).  Y (bf16, f16 or fp32, contiguous:
 * ldy == N) is bit-identical to df_fp8_gemm_fwd's.  *y_absmax_dev gets the
 * absmax over the finite values of Y as stored, and *y_scale_dev the rule-D1/D2
 * scale for next_fmt, exactly what df_absmax_scale_bf16 / _f16 / _f32 give on Y
 * (either output may be NULL, not both).  On the unsplit 256x256 plan the
 * kernel folds |Y| in its epilogue and one block folds the partials, so Y
 * is not read again; other plans run the two passes.  ws:
 * df_fp8_gemm_fwd_absmax_workspace_bytes(M, N, K) for the fused kernel; at
 * least df_absmax_workspace_bytes() runs the two passes.  Calls that overlap
 * on one workspace race. */
size_t df_fp8_gemm_fwd_absmax_workspace_bytes(int M, int N, int K);
int df_fp8_gemm_fwd_absmax(const uint8_t* Xq, int ldx, const uint8_t* Wq, int ldw, int M, int N, int K,
                           const float* sx_dev, const float* sw_dev, int bias_dtype, const void* bias,
                           int y_dtype, void* Y, int ldy, int next_fmt, float* y_absmax_dev,
                           float* y_scale_dev, void* ws, size_t ws_bytes, void* stream);
/* dX[M,K] = dY_q[M,N] . W[N,K]  (e5m2 x e4m3), given W^T quantized as
 * Wt_q[K, ldwt] (df_quantize_2d's qt).  Replaces fc_backward_input
 * (fully_connected_layer.cu:43-65). */
int df_fp8_gemm_bwd_dx(const uint8_t* dYq, int lddy, const uint8_t* Wtq, int ldwt,
                       int M, int N, int K, const float* sdy_dev, const float* sw_dev,
                       int dx_dtype, void* dX, int lddx,
                       void* ws, size_t ws_bytes, void* stream);
/* dW[N,K] = dY^T . X, given dY^T quantized as dYt_q[N, ldyt] (e5m2) and X^T
 * as Xt_q[K, ldxt] (e4m3); M tokens is the reduction.  Overwrites dW, like
 * fc_backward_weights (fully_connected_layer.cu:67-89, :85-87). */
int df_fp8_gemm_bwd_dw(const uint8_t* dYtq, int ldyt, const uint8_t* Xtq, int ldxt,
                       int M, int N, int K, const float* sdy_dev, const float* sx_dev,
                       int dw_dtype, void* dW, int lddw,
                       void* ws, size_t ws_bytes, void* stream);
/* dX and dW of one Linear in one launch: the arguments of df_fp8_gemm_bwd_dx
 * and df_fp8_gemm_bwd_dw together (M tokens, N outputs, K inputs).  The dW
 * GEMM has few output tiles (6400 x 1600: 175 of 256 x 256 for 256 CUs), so
 * its launch alone leaves CUs idle; here one persistent grid takes dW's work
 * units first and deals dX's tiles to the CUs as they free up (a static
 * schedule, no atomics).  dX is bit-identical to df_fp8_gemm_bwd_dx (where
 * that call would cut dX's reduction into K slices, the two calls are made
 * instead of the grouped launch); dW to
 * df_fp8_gemm_bwd_dw whenever both split its K range alike (they may pick
 * different slice counts, which changes dW's fp32 rounding, within the
 * 1e-4 bar either way).  Falls back to the two calls where the grouped
 * launch does not apply (degenerate sizes, operands beyond 2^31 bytes, a
 * HALF output paired with a non-HALF one) or would not be faster.  ws: df_fp8_gemm_bwd_workspace_bytes(M, N, K) never
 * limits the plan; smaller only narrows it.  Together these replace
 * fc_backward_input and fc_backward_weights (fully_connected_layer.cu:43-89)
 * as FullyConnectedLayer::backward launches them (:310-338). */
size_t df_fp8_gemm_bwd_workspace_bytes(int M, int N, int K);
/* The plan df_fp8_gemm_bwd takes for these sizes, a workspace of ws_bytes
 * and operands with the smallest leading dimensions: *grouped = 1 for the
 * one grouped launch (then *dw_slices = the K slices of dW, 1 = unsplit),
 * 0 for the two separate calls (*dw_slices = 0). */
int df_fp8_gemm_bwd_plan(int M, int N, int K, size_t ws_bytes, int* grouped, int* dw_slices);
int df_fp8_gemm_bwd(const uint8_t* dYq, int lddy, const uint8_t* Wtq, int ldwt,
                    const uint8_t* dYtq, int ldyt, const uint8_t* Xtq, int ldxt,
                    int M, int N, int K, const float* sdy_dev, const float* sw_dev,
                    const float* sx_dev, int dx_dtype, void* dX, int lddx,
                    int dw_dtype, void* dW, int lddw,
                    void* ws, size_t ws_bytes, void* stream);
/* df_fp8_gemm_bwd whose dX also gives the absmax the upstream Linear's
 * just-in-time dY scale needs (new; no counterpart in the reference, whose
 * TransformerBlock backward passes fc2's input gradient straight to fc1 as
 * its output gradient, dnn/layers/transformer_block.cu:127-134).  dX (bf16,
 * f16 or fp32, contiguous: lddx == K, 16-byte aligned) and dW are bit-identical
 * to df_fp8_gemm_bwd's with a workspace of df_fp8_gemm_bwd_workspace_bytes.
 * *dx_absmax_dev gets the absmax over the finite values of dX as stored and
 * *dx_scale_dev the rule-D1/D2 scale for next_fmt (either may be NULL, not
 * both): what df_absmax_scale_bf16 / _f16 / _f32 give on dX.  When the plan
 * is the grouped launch (an f16 dX groups with an f16 dW only), its dX
 * tiles fold |dX| in their epilogue and one block folds the partials;
 * otherwise dX is read again by the absmax pass.  ws:
 * df_fp8_gemm_bwd_absmax_workspace_bytes(M, N, K) (its first part holds the
 * partials, the rest is df_fp8_gemm_bwd's workspace). */
size_t df_fp8_gemm_bwd_absmax_workspace_bytes(int M, int N, int K);
int df_fp8_gemm_bwd_absmax(const uint8_t* dYq, int lddy, const uint8_t* Wtq, int ldwt,
                           const uint8_t* dYtq, int ldyt, const uint8_t* Xtq, int ldxt,
                           int M, int N, int K, const float* sdy_dev, const float* sw_dev,
                           const float* sx_dev, int dx_dtype, void* dX, int lddx,
                           int dw_dtype, void* dW, int lddw, int next_fmt,
                           float* dx_absmax_dev, float* dx_scale_dev,
                           void* ws, size_t ws_bytes, void* stream);

/* ---- layer weight streaming (new: the reference describes layer-serialized
 * execution, README.md:212-226, and has its host-side pieces in the NVMe
 * loader -- pinned cudaHostAlloc buffers, per-slot streams, cudaMemcpyAsync,
 * apps/host-multi/NVMeLoader_Linux.hpp:20-26,64-71,123-125) ----
 * A streamer owns `slots` device buffers of slot_bytes (rounded up to 4 KiB)
 * and two copy streams of default priority (consecutive loads alternate, so
 * one copy's start overlaps the other's transfer).  Per layer:
 *   df_streamer_load    : blocks the calling thread until the work recorded
 *                         by the next slot's last df_streamer_release has
 *                         completed, then enqueues the copy of `bytes` from
 *                         host memory (pinned, for the copy to be
 *                         asynchronous) into that slot (ring order) on a
 *                         copy stream;
 *   df_streamer_wait    : makes `stream` wait until the slot's copy landed;
 *   df_streamer_release : records, on `stream`, the point after which the
 *                         slot may be overwritten (call it after enqueuing
 *                         every launch that reads the slot).
 * Issue load(l + slots - 2) right after layer l's launches: the thread then
 * blocks only until layer l-2 has finished, with layers l-1 and l queued.
 * Loading into a slot that was loaded but not released is DF_ERR_INVALID.
 * One streamer is used by one host thread at a time.  The streamer is driven
 * from the host (df_streamer_load waits on events there), so it is not for
 * use inside HIP graph capture; the GEMM and quantize calls of each layer
 * are. */
typedef struct df_streamer_s df_streamer;
int df_host_alloc(size_t bytes, void** host_ptr);  /* pinned host memory (hipHostMalloc) */
int df_host_free(void* host_ptr);
int df_streamer_create(int slots, size_t slot_bytes, df_streamer** out);
int df_streamer_destroy(df_streamer* s);             /* waits for its copies first */
int df_streamer_load(df_streamer* s, const void* host_src, size_t bytes, int* slot, void** dev_ptr);
int df_streamer_wait(df_streamer* s, int slot, void* stream);
int df_streamer_release(df_streamer* s, int slot, void* stream);
int df_streamer_slot(df_streamer* s, int slot, void** dev_ptr);
/* copy stream `which` (0 or 1): load i is enqueued on copy stream i % 2, so
 * a caller that synchronizes with the copies needs both */
int df_streamer_copy_stream(df_streamer* s, int which, void** stream);
/* Timing of the copies (new; no counterpart in the reference): with timing
 * on, each load records a HIP event on its copy stream right before and
 * right after the copy.  df_streamer_copy_log waits for every timed copy,
 * writes up to `capacity` (start, end) pairs in load order -- ms after an
 * event recorded just before the first timed copy since the log was last
 * read -- sets *count to the number logged, and clears the log when all of them
 * fit in `capacity` (capacity 0: a query of the count).  A copy's
 * start is when its copy stream reached it (the previous copy on that
 * stream had finished); with two streams, two copies can share the link
 * between those marks. */
int df_streamer_set_timing(df_streamer* s, int on);
int df_streamer_copy_log(df_streamer* s, float* start_ms, float* end_ms, int capacity, int* count);

/* ---- consumer side of the fp32 gradients: global-norm clipping and Adam ----
 * Lists of fp32 tensors: the pointer arrays and `sizes` are HOST arrays of
 * `count` entries holding DEVICE pointers (16-byte aligned) and element
 * counts; zero-size entries are skipped.
 *
 * df_grad_norm_f32 writes norm_dev[0] = sqrt(sum over every element of
 * RN32(g*g)), the squares accumulated in binary64 in a fixed order, the root
 * rounded once to binary32.  It replaces the host-side norm of
 * utils::clip_grad_norm (dnn/utils/clip_grad_norm.cu:31-50), which downloads
 * every gradient and sums in binary32.  `ws` holds
 * df_grad_norm_workspace_bytes(count, sizes) bytes (8-byte aligned).
 *
 * df_clip_grad_norm_f32 is utils::clip_grad_norm (clip_grad_norm.cu:31-67):
 * the norm as above, then every element g = g * (max_norm / norm) when
 * norm > max_norm, decided on the device (no host synchronisation).
 *
 * df_adam_update_f32 is one AdamOptimizer<float>::step over the list
 * (dnn/optimizers/adam_optimizer.cu:83-109 with adam_update_kernel's float
 * path, :24-30), `timestep` the already-incremented step count (>= 1):
 *   g = grad + wd*p;  m = b1*m + (1-b1)*g;  v = b2*v + (1-b2)*g*g;
 *   p = p - lr * (m / (1 - b1^t)) / (sqrt(v / (1 - b2^t)) + eps)
 * every operation rounded to binary32 (no fused multiply-add), IEEE division
 * and square root; b^t is rounded to binary32 on the host.  With
 * clip_norm_dev non-NULL, grad is first multiplied by max_norm / norm when
 * norm = clip_norm_dev[0] > max_norm: the same values as
 * df_clip_grad_norm_f32 followed by this call, without rewriting the
 * gradients.  Under HIP graph capture, lr and the two bias corrections
 * (from `timestep`) are fixed when the call is captured (they are kernel
 * arguments): every replay repeats that step's values. */
size_t df_grad_norm_workspace_bytes(int count, const int64_t* sizes);
int df_grad_norm_f32(const float* const* grads, const int64_t* sizes, int count,
                     float* norm_dev, void* ws, size_t ws_bytes, void* stream);
int df_clip_grad_norm_f32(float* const* grads, const int64_t* sizes, int count,
                          float max_norm, float* norm_dev, void* ws, size_t ws_bytes,
                          void* stream);
int df_adam_update_f32(float* const* params, const float* const* grads, float* const* m,
                       float* const* v, const int64_t* sizes, int count, float lr,
                       float beta1, float beta2, float eps, float weight_decay,
                       int timestep, const float* clip_norm_dev, float max_norm,
                       void* stream);
/* df_adam_update_f32 that also writes absmax_dev[i] (device array of
 * `count` floats) = max |p| over the finite values of the updated
 * parameters of tensor i (0 for an empty one): the absmax the next step's
 * quantization of the weights needs, measured while the update already
 * holds them in registers instead of in a pass of its own over every
 * parameter.  The parameters, m and v are bit-identical to
 * df_adam_update_f32's.  No reference counterpart (the reference has no fp8
 * weights); pair it with df_quantize_2d_batch_absmax. */
int df_adam_update_absmax_f32(float* const* params, const float* const* grads, float* const* m,
                              float* const* v, const int64_t* sizes, int count, float lr,
                              float beta1, float beta2, float eps, float weight_decay,
                              int timestep, const float* clip_norm_dev, float max_norm,
                              float* absmax_dev, void* stream);

/* ---- tensor utilities behind dnn::tensor (dnn/core/tensor.cu:18-52) ---- */
/* fill_kernel (tensor.cu:19): n elements of elem_bytes (1, 2 or 4) = *value */
int df_fill(void* dst, int64_t n, int elem_bytes, const void* value_host, void* stream);
/* add_kernel / add_inplace_kernel (tensor.cu:27-36): out = a + b (out may be a) */
int df_add(int dtype, const void* a, const void* b, void* out, int64_t n, void* stream);
/* equal_kernel (tensor.cu:39): mask[i] = bitwise a[i] == b[i] (per element) */
int df_equal_mask(int dtype, const void* a, const void* b, uint8_t* mask, int64_t n,
                  void* stream);
/* elementwise cast, the reference's utils::to_float / to_half
 * (dnn/utils/convert.cu:6-27) as a tensor op: fp32 -> bf16, fp32 -> f16,
 * bf16 -> f16 (round to nearest even once, from the exact binary32 value;
 * f16 subnormals kept, |x| >= 65520 -> inf; NaN -> sign|0x7FC0 (bf16) or
 * sign|0x7E00 (f16)); bf16, f16, int8 -> fp32 and int8 -> f16 (exact; a
 * NaN keeps its payload); fp32 -> fp32 (a copy).  Other pairs:
 * DF_ERR_UNSUPPORTED. */
int df_convert(int in_dtype, const void* in, int out_dtype, void* out, int64_t n, void* stream);
/* approx_equal_kernel (tensor.cu:46): mask[i] = |a[i]-b[i]| <= atol, in fp32 */
int df_approx_equal_mask(int dtype, const void* a, const void* b, uint8_t* mask,
                         int64_t n, float atol, void* stream);

#ifdef __cplusplus
}
#endif
#endif
