/*
 * df_oracle.h -- CPU restatement of the fp8 Linear path (TEST INFRASTRUCTURE).
 *
 * This library is the checker for the HIP product path, never part of it.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product library (libdeepfuse_amd.so) does not link it and
 * must fail loudly when its own HIP code is missing.
 *
 * What each group of functions follows:
 *
 *  - fp8 codec: the OCP 8-bit Floating Point specification (OFP8) v1.0.
 *    The reference has no conversion code: fp8 appears there only as the
 *    packed types instantiated at dnn/core/tensor.cu:489-498 (guarded by
 *    __CUDA_FP8_TYPES_EXIST__, dnn/core/tensor.cuh:7-9) and the claim at
 *    README.md:16.  The contract decisions this restatement pins:
 *      D1  s = absmax / FMAX in binary32; q = sat_rne(x / s), IEEE division.
 *      D2  absmax over finite values only; absmax == 0 or a scale that is
 *          not a positive finite number gives s = 1.
 *      D3  NaN -> sign|0x7F (e4m3 and e5m2); +-inf -> +-max finite
 *          (e4m3 0x7E/0xFE = 448, e5m2 0x7B/0xFB = 57344); finite values
 *          beyond max saturate.
 *      D4  fp32 subnormals are honoured (no flush to zero).
 *      D5  dequantized value = decode(q) * s in binary32 (RN); bf16 output is
 *          the RNE rounding of that binary32; a NaN code dequantizes to the
 *          canonical quiet NaN 0x7FC00000 (bf16 0x7FC0) with the code's sign.
 *
 *  - FC loops: dnn/layers/fully_connected_layer.cu, kernel order:
 *      forward  :29-35  sum_k x*w sequential in fp32, then + bias
 *      dX       :54-59  sum over out-features sequential
 *      dW       :78-83  sum over tokens sequential, overwrite
 *      db       :99-101 sum over tokens sequential
 *    and the GTest host oracle tests/layers/fully_connected_layer_test.cu:29-46
 *    (bias first, then accumulate), used as a second CPU baseline variant.
 *
 * Parity pins (where each function is checked; see tests/test_oracle_*.py):
 *    codec encode : exhaustive 2^32 fp32 sweep against a nearest-code table
 *                   search with ties-to-even (independent method), torch CPU
 *                   float8 casts after clamping, golden vectors.
 *    codec decode : closed form from the spec, all 256 codes, torch casts.
 *    absmax/scale : brute force, order independence, NaN/inf exclusion.
 *    quantize     : x/s then encode; golden KAT from the reference FC test.
 *    FC loops     : reference KAT y={5.5,10.5} (fully_connected_layer_test.cu
 *                   :266-284), numpy float64 products, closed forms.
 *    grad norm    : closed forms (sqrt(n) for ones, 3-4-5), numpy binary64
 *                   pairwise sums, the reference's binary32 host sum on
 *                   exactly summable inputs and within its error bound.
 *    clip         : no scaling at norm <= max_norm, clipped norm == max_norm
 *                   within rounding, factor applied elementwise.
 *    Adam         : the reference's GTest expectations
 *                   (tests/optimizers/adam_optimizer_test.cu:21-214), the
 *                   two-step closed form m_hat = (b1 g1 + g2)/(1 + b1),
 *                   v_hat = (b2 g1^2 + g2^2)/(1 + b2), the constant-gradient
 *                   fixed point, coupled (L2) weight decay, exact powers of
 *                   two for the bias correction.
 */
#ifndef DF_ORACLE_H
#define DF_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Format selector, same values as the product's DF_FMT_* (df_capi.h). */
enum { DFO_E4M3 = 0, DFO_E5M2 = 1 };

/* ---- scalar codec ---- */
uint8_t dfo_encode(float v, int fmt);          /* RNE, saturating, D3 */
float dfo_decode(uint8_t q, int fmt);          /* exact; NaN code -> canonical qNaN */
float dfo_fmax(int fmt);                       /* 448 or 57344 */
uint16_t dfo_f32_to_bf16(float v);             /* RNE; NaN -> sign|0x7FC0 */
float dfo_bf16_to_f32(uint16_t h);             /* exact widening */
/* binary32 <-> IEEE binary16, the reference's utils::to_half / to_float
 * (dnn/utils/convert.cu:6-27): RNE narrowing with subnormals, |v| >= 65520
 * -> inf, NaN -> sign|0x7E00; exact widening, NaN payload kept. */
uint16_t dfo_f32_to_f16(float v);
float dfo_f16_to_f32(uint16_t h);
/* Arrays of DType 0 (binary32), 1 (binary16), 2 (int8, input only) or 4
 * (bf16): exact widening to binary32, then one rounding to the output type;
 * -1 for an unsupported pair. */
int dfo_convert(int in_dtype, const void* in, int out_dtype, void* out, int64_t n);

/* ---- tensor ops ---- */
float dfo_absmax_f32(const float* x, int64_t n);           /* D2 */
float dfo_absmax_bf16(const uint16_t* x, int64_t n);
float dfo_scale(float absmax, int fmt);                    /* D1/D2 */
void dfo_quantize_f32(const float* x, int64_t n, float s, int fmt, uint8_t* q);
void dfo_quantize_bf16(const uint16_t* x, int64_t n, float s, int fmt, uint8_t* q);
void dfo_dequantize_f32(const uint8_t* q, int64_t n, float s, int fmt, float* out);
void dfo_dequantize_bf16(const uint8_t* q, int64_t n, float s, int fmt, uint16_t* out);

/* Encode of every fp32 bit pattern in [first, first+count) at s = 1:
 * the exhaustive sweep helper (nthreads <= 0 -> one thread). */
void dfo_encode_bits_range(uint32_t first, int64_t count, int fmt, uint8_t* out,
                           int nthreads);

/* bf16 (to_f16 == 0) or binary16 (to_f16 != 0) narrowing of every fp32 bit
 * pattern in [first, first+count) (exhaustive conversion sweeps). */
void dfo_narrow_bits_range(uint32_t first, int64_t count, int to_f16, uint16_t* out,
                           int nthreads);

/* Independent encoder for the exhaustive pin: binary search of the sorted
 * table of non-negative finite codes, nearest value, ties to the even code,
 * beyond max saturates.  Shares no code with dfo_encode. */
uint8_t dfo_encode_by_table(float v, int fmt);
/* Number of fp32 patterns in [first, first+count) where the two encoders
 * disagree (first mismatch's pattern in *first_bad when non-null). */
int64_t dfo_sweep_compare(uint32_t first, int64_t count, int fmt,
                          uint32_t* first_bad, int nthreads);

/* ---- FC loops (row-major; W is [out, in]) ---- */
void dfo_fc_forward(const float* X, const float* W, const float* b, float* Y,
                    int N, int in_f, int out_f, int nthreads);
void dfo_fc_forward_bias_first(const float* X, const float* W, const float* b,
                               float* Y, int N, int in_f, int out_f, int nthreads);
void dfo_fc_backward_input(const float* dY, const float* W, float* dX,
                           int N, int in_f, int out_f, int nthreads);
void dfo_fc_backward_weights(const float* dY, const float* X, float* dW,
                             int N, int in_f, int out_f, int nthreads);
void dfo_fc_backward_bias(const float* dY, float* db, int N, int out_f);

/* ---- consumer side: global-norm clipping and Adam ----
 * Follows dnn/utils/clip_grad_norm.cu:13-67 and the float path of
 * dnn/optimizers/adam_optimizer.cu:11-30,83-109. */
double dfo_sumsq(const float* x, int64_t n);                  /* sum RN32(x*x), binary64 */
float dfo_grad_norm(const float* const* g, const int64_t* n, int count);
float dfo_grad_norm_ref_f32(const float* const* g, const int64_t* n, int count);
int dfo_clip_scale(float* g, int64_t n, float norm, float max_norm);
float dfo_bias_correction(float beta, int t);                 /* 1 - RN32(beta^t) */
void dfo_adam_step(float* p, const float* grad, float* m, float* v, int64_t n,
                   float lr, float beta1, float beta2, float eps, float wd, int t,
                   float clip_factor);

/* ---- delayed scaling: push amax into history[0..len) (newest first) and
 * return the scale of the new maximum, the one the next pass uses ---- */
float dfo_history_push(float* history, int len, float amax, int fmt);

/* ---- LayerNorm forward (dnn/layers/layer_norm_layer.cu:26-63), per row of
 * C; gamma/beta NULL = no affine map; round_bf16 rounds y to bf16 ---- */
void dfo_layernorm(const float* x, int rows, int C, const float* gamma, const float* beta,
                   float eps, int round_bf16, float* y);

#ifdef __cplusplus
}
#endif
#endif
