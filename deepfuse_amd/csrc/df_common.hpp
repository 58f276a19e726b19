// df_common.hpp -- shared host/device helpers for libdeepfuse_amd (gfx950).
//
// Device side: the OCP OFP8 v1.0 codec (e4m3 / e5m2), round-to-nearest-even
// and saturating, written for the VALU (integer-domain significand rounding,
// one v_rndne for subnormal targets), plus bf16 rounding.  The contract it
// implements (scale rule, NaN/inf policy, subnormals) is the one stated at the
// top of include/df_capi.h.
//
// Host side: the thread-local error string behind df_last_error_string() and
// the argument-check macros every C-ABI entry point uses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/df_capi.h"

namespace dfk {

// native clang vectors (the nontemporal builtins take these, not HIP's
// HIP_vector_type wrappers)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- formats --
enum : int { E4M3 = DF_FMT_E4M3, E5M2 = DF_FMT_E5M2 };

template <int FMT> struct Fp8;
template <> struct Fp8<E4M3> {
    static constexpr int mbits = 3, bias = 7;
    static constexpr uint32_t max_bits = 0x43E00000u;  // 448.0f
    static constexpr uint32_t max_code = 0x7Eu;
    static constexpr float fmax = 448.0f;
};
template <> struct Fp8<E5M2> {
    static constexpr int mbits = 2, bias = 15;
    static constexpr uint32_t max_bits = 0x47600000u;  // 57344.0f
    static constexpr uint32_t max_code = 0x7Bu;
    static constexpr float fmax = 57344.0f;
};

// ------------------------------------------------------------ absmax fold --
// |x| over finite values as an unsigned max of the sign-cleared bit patterns
// (monotone for non-negative binary32); inf/NaN patterns (>= 0x7F800000)
// contribute 0.
__device__ __forceinline__ uint32_t fold_f32(uint32_t m, uint32_t bits) {
    const uint32_t a = bits & 0x7FFFFFFFu;
    return max(m, a < 0x7F800000u ? a : 0u);
}

// two bf16 in one dword: widen each to its binary32 pattern
__device__ __forceinline__ uint32_t fold_bf16x2(uint32_t m, uint32_t w) {
    const uint32_t hi = w & 0x7FFF0000u;
    const uint32_t lo = (w << 16) & 0x7FFF0000u;
    m = max(m, hi < 0x7F800000u ? hi : 0u);
    return max(m, lo < 0x7F800000u ? lo : 0u);
}

// The same folds without compares, for code whose VALU slots are scarce (a
// compare's lane mask read by the next VALU instruction costs wait states).
// Adding 0x00800000 to a sign-cleared binary32 pattern (0x0080 to each
// sign-cleared bf16 half of a dword: no carry crosses the halves) maps finite
// patterns to positive and inf/NaN patterns to negative signed values, so a
// signed max that starts at 0 skips the latter.  unbias_* turns such an
// accumulator back into the binary32 pattern fold_f32 / fold_bf16x2 give.
__device__ __forceinline__ uint32_t fold_f32_biased(uint32_t m, uint32_t bits) {
    return (uint32_t)max((int)m, (int)((bits & 0x7FFFFFFFu) + 0x00800000u));
}
__device__ __forceinline__ uint32_t unbias_f32(uint32_t m) { return (uint32_t)max((int)m - 0x00800000, 0); }

typedef short df_short2 __attribute__((ext_vector_type(2)));
// two bf16 in one dword, one 16-bit lane each (v_pk_max_i16)
__device__ __forceinline__ uint32_t fold_bf16x2_biased(uint32_t m, uint32_t w) {
    const df_short2 u = __builtin_bit_cast(df_short2, (w & 0x7FFF7FFFu) + 0x00800080u);
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(df_short2, m), u));
}
__device__ __forceinline__ uint32_t unbias_bf16x2(uint32_t m) {
    const int hi = (int)(int16_t)(m >> 16), lo = (int)(int16_t)(m & 0xFFFFu);
    return (uint32_t)max(max(hi, lo) - 0x80, 0) << 16;
}

// ----------------------------------------------------------------- encode --
// binary32 -> fp8 code in the low byte.  |v| >= max (inf included) saturates,
// NaN gives sign|0x7F.  Normal targets round the re-biased significand in
// the integer domain; subnormal targets scale by 2^(bias-1+mbits) (exact)
// and round to an integer with v_rndne_f32.
template <int FMT>
__device__ __forceinline__ uint32_t encode_fp8(float v) {
    using T = Fp8<FMT>;
    constexpr int sh = 23 - T::mbits;
    constexpr uint32_t min_normal_bits = (uint32_t)(128 - T::bias) << 23;
    constexpr float sub_scale = (float)(1u << (T::bias - 1 + T::mbits));
    const uint32_t u = __float_as_uint(v);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7FFFFFFFu;
    const uint32_t ac = a < T::max_bits ? a : T::max_bits;
    uint32_t r = ac - ((uint32_t)(127 - T::bias) << 23);
    r = (r + ((1u << (sh - 1)) - 1u) + ((r >> sh) & 1u)) >> sh;
    const uint32_t rs = (uint32_t)__builtin_rintf(__uint_as_float(ac) * sub_scale);
    uint32_t code = ac < min_normal_bits ? rs : r;
    code = a > 0x7F800000u ? 0x7Fu : code;
    return code | sign;
}

// ------------------------------------------------------- x / s, exactly --
// Quantization divides every element by the same scale s, so the kernels
// use the reciprocal r = RN(1/s) (one IEEE division per thread) and
// Markstein's correction: y0 = RN(x*r); one fma refinement makes y1 a
// faithful quotient, whose remainder e1 = x - s*y1 is exact (fma), and
// RN(y1 + e1*r) is then the correctly rounded x/s (Markstein's theorem:
// faithful quotient + correctly rounded reciprocal, no over/underflow).
// The fast form is used only when 2^-40 <= s <= 2^40, for |x| <= 2^60:
//  - quotients stay below 2^100, so nothing overflows;
//  - a quotient that can round to a non-zero fp8 code (|x/s| >= 2^-17) has
//    |x| >= 2^-57, which keeps products and remainders clear of binary32
//    underflow (exact remainders need |x| >= 2^-102);
//  - |x| > 2^60 (inf included) means |x/s| > 2^20, beyond both formats'
//    maximum, so x itself goes to the saturating encoder.
// NaN inputs pass through with their sign; s > 0, so the quotient carries
// x's sign, which copysign restores for -0 (the fma chain gives +0).
// Other scales use the IEEE division x / s.
struct QDiv {
    float s, r;
    bool fast;
};

__device__ __forceinline__ QDiv make_qdiv(float s) {
    QDiv d;
    d.s = s;
    d.r = 1.0f / s;
    d.fast = s >= 0x1p-40f && s <= 0x1p40f;
    return d;
}

// FAST selects the form at compile time: kernels test d.fast once and run a
// loop instantiated for it, so no per-element branch splits their code.
template <bool FAST>
__device__ __forceinline__ float qdiv_t(float x, const QDiv& d) {
    if (!FAST) return x / d.s;
    const float y0 = x * d.r;
    const float e0 = __builtin_fmaf(-d.s, y0, x);
    const float y1 = __builtin_fmaf(e0, d.r, y0);
    const float e1 = __builtin_fmaf(-d.s, y1, x);
    const float q = __builtin_copysignf(__builtin_fmaf(e1, d.r, y1), x);
    return __builtin_fabsf(x) <= 0x1p60f ? q : x;  // NaN and huge inputs pass through
}

__device__ __forceinline__ float qdiv(float x, const QDiv& d) {
    return d.fast ? qdiv_t<true>(x, d) : qdiv_t<false>(x, d);
}

// Two values -> two fp8 codes with the hardware converter
// (v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32: round to nearest even).  Inputs are
// clamped to +-max first (saturation, inf included) and NaN gets the
// sign|0x7F code explicitly; this form was compared with encode_fp8 on all
// 2^32 binary32 inputs for both formats and agrees everywhere.
template <int FMT>
__device__ __forceinline__ uint32_t encode2_hw(float a, float b) {
    constexpr float fm = Fp8<FMT>::fmax;
    const float ca = __builtin_fminf(__builtin_fmaxf(a, -fm), fm);
    const float cb = __builtin_fminf(__builtin_fmaxf(b, -fm), fm);
    uint32_t p = (uint32_t)(FMT == E4M3 ? __builtin_amdgcn_cvt_pk_fp8_f32(ca, cb, 0, false)
                                        : __builtin_amdgcn_cvt_pk_bf8_f32(ca, cb, 0, false)) & 0xFFFFu;
    const uint32_t ua = __float_as_uint(a), ub = __float_as_uint(b);
    if ((ua & 0x7FFFFFFFu) > 0x7F800000u) p = (p & 0xFF00u) | ((ua >> 24) & 0x80u) | 0x7Fu;
    if ((ub & 0x7FFFFFFFu) > 0x7F800000u) p = (p & 0x00FFu) | ((((ub >> 24) & 0x80u) | 0x7Fu) << 8);
    return p;
}

// four elements x / s -> four packed codes (byte i = element i)
template <int FMT, bool FAST>
__device__ __forceinline__ uint32_t quant4_t(float a, float b, float c, float d, const QDiv& q) {
    return encode2_hw<FMT>(qdiv_t<FAST>(a, q), qdiv_t<FAST>(b, q)) |
           (encode2_hw<FMT>(qdiv_t<FAST>(c, q), qdiv_t<FAST>(d, q)) << 16);
}

// The same codes for inputs known not to be NaN, fast division form only
// (kernels test a group of values with one wave-wide ballot and take
// quant4_t when any lane holds a NaN).  About half the instructions:
//  - |x| above 2^60 (inf included) is clamped to 2^60 before the division
//    instead of selected around it: the quotient is then above 2^20, beyond
//    both formats' maximum, and saturates to the same code;
//  - the clamp to +-max is one v_med3 (no NaN to canonicalise first), and
//    no NaN patch follows the conversion;
//  - the second pair of codes is converted into the high half of the first
//    pair's register (word select) instead of being masked and shifted.
// med3 returns one of its operands, so -0 stays -0 through both clamps.
template <int FMT>
__device__ __forceinline__ float qdiv_clamp_nonan(float x, const QDiv& d) {
    const float xc = __builtin_amdgcn_fmed3f(x, -0x1p60f, 0x1p60f);
    const float y0 = xc * d.r;
    const float e0 = __builtin_fmaf(-d.s, y0, xc);
    const float y1 = __builtin_fmaf(e0, d.r, y0);
    const float e1 = __builtin_fmaf(-d.s, y1, xc);
    const float q = __builtin_copysignf(__builtin_fmaf(e1, d.r, y1), x);
    constexpr float fm = Fp8<FMT>::fmax;
    return __builtin_amdgcn_fmed3f(q, -fm, fm);
}

template <int FMT>
__device__ __forceinline__ uint32_t quant4_nonan(float a, float b, float c, float d, const QDiv& q) {
    const float qa = qdiv_clamp_nonan<FMT>(a, q), qb = qdiv_clamp_nonan<FMT>(b, q);
    const float qc = qdiv_clamp_nonan<FMT>(c, q), qd = qdiv_clamp_nonan<FMT>(d, q);
    if (FMT == E4M3)
        return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(qc, qd, __builtin_amdgcn_cvt_pk_fp8_f32(qa, qb, 0, false),
                                                         true);
    return (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(qc, qd, __builtin_amdgcn_cvt_pk_bf8_f32(qa, qb, 0, false),
                                                     true);
}

// True when any lane of the wave holds a NaN among v[0..N-1] (uniform).
template <int N>
__device__ __forceinline__ bool wave_any_nan(const float* v) {
    uint64_t m = 0;
#pragma unroll
    for (int e = 0; e < N; ++e) m |= __builtin_amdgcn_ballot_w64(v[e] != v[e]);
    return m != 0;
}

// Four packed codes per row for rows a..d -> the four columns (byte i of
// column j = byte j of row i): a 4x4 byte transpose in eight v_perm_b32.
__device__ __forceinline__ void transpose4x4_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t* col) {
    const uint32_t ab01 = __builtin_amdgcn_perm(b, a, 0x05010400u);  // a0 b0 a1 b1
    const uint32_t cd01 = __builtin_amdgcn_perm(d, c, 0x05010400u);  // c0 d0 c1 d1
    const uint32_t ab23 = __builtin_amdgcn_perm(b, a, 0x07030602u);  // a2 b2 a3 b3
    const uint32_t cd23 = __builtin_amdgcn_perm(d, c, 0x07030602u);  // c2 d2 c3 d3
    col[0] = __builtin_amdgcn_perm(cd01, ab01, 0x05040100u);          // a0 b0 c0 d0
    col[1] = __builtin_amdgcn_perm(cd01, ab01, 0x07060302u);          // a1 b1 c1 d1
    col[2] = __builtin_amdgcn_perm(cd23, ab23, 0x05040100u);
    col[3] = __builtin_amdgcn_perm(cd23, ab23, 0x07060302u);
}

// ----------------------------------------------------------------- decode --
// fp8 code (low byte) -> binary32, exact.  The magnitude bits shifted into
// the binary32 exponent/significand position are the value times
// 2^-(127-bias) for normal and subnormal codes alike (binary32 subnormals
// are honoured), so one multiply by 2^(127-bias) restores it.
template <int FMT>
__device__ __forceinline__ float decode_fp8(uint32_t q) {
    using T = Fp8<FMT>;
    constexpr float up = (FMT == E4M3) ? 0x1p120f : 0x1p112f;
    const uint32_t mag = q & 0x7Fu;
    const uint32_t sign = (q & 0x80u) << 24;
    float v = __uint_as_float(mag << (23 - T::mbits)) * up;
    uint32_t bits = __float_as_uint(v) | sign;
    if (FMT == E4M3) {
        bits = mag == 0x7Fu ? (sign | 0x7FC00000u) : bits;
    } else {
        bits = mag == 0x7Cu ? (sign | 0x7F800000u) : bits;
        bits = mag > 0x7Cu ? (sign | 0x7FC00000u) : bits;
    }
    return __uint_as_float(bits);
}

// dequantized value: decode(q) * s, NaN codes -> canonical quiet NaN.
template <int FMT>
__device__ __forceinline__ float dequant_fp8(uint32_t q, float s) {
    const uint32_t mag = q & 0x7Fu;
    const bool is_nan = (FMT == E4M3) ? (mag == 0x7Fu) : (mag > 0x7Cu);
    const float v = decode_fp8<FMT>(q) * s;
    return is_nan ? __uint_as_float(((q & 0x80u) << 24) | 0x7FC00000u) : v;
}

// ------------------------------------------------------------------- bf16 --
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
    return (u & 0x7FFFFFFFu) > 0x7F800000u ? (((u >> 16) & 0x8000u) | 0x7FC0u) : r;
}
__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// --------------------------------------------------------------- binary16 --
// binary32 -> IEEE binary16 with the hardware convert (v_cvt_f16_f32: round
// to nearest even under the default mode, binary16 subnormals kept, |x| >=
// 65520 -> inf); NaN gives the quiet NaN sign|0x7E00, the policy of the
// bf16 rounding above.
__device__ __forceinline__ uint32_t f32_to_f16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)f);
    return (u & 0x7FFFFFFFu) > 0x7F800000u ? (((u >> 16) & 0x8000u) | 0x7E00u) : h;
}
// binary16 -> binary32, exact; a NaN keeps its sign and payload bits (the
// hardware convert would set the quiet bit of a signalling NaN).
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    const float v = (float)__builtin_bit_cast(_Float16, (uint16_t)h);
    const bool nan = (h & 0x7C00u) == 0x7C00u && (h & 0x03FFu) != 0u;
    return nan ? __uint_as_float(((h & 0x8000u) << 16) | 0x7F800000u | ((h & 0x03FFu) << 13)) : v;
}

// A binary16 element in kernel templates: the storage of DF_DTYPE_HALF,
// distinct from uint16_t, which there always holds bf16 bits.
struct f16_t {
    uint16_t bits;
};
static_assert(sizeof(f16_t) == 2, "f16_t is two bytes");

// The biased fold above for two binary16 values: |x| + 0x0400 takes +inf
// and every NaN (0x7C00 and up) to a negative int16, which the signed max
// skips; finite values keep their order.  unbias_f16x2 gives the binary32
// bits of the largest finite |x| folded (0 if none).
__device__ __forceinline__ uint32_t fold_f16x2_biased(uint32_t m, uint32_t w) {
    const df_short2 u = __builtin_bit_cast(df_short2, (w & 0x7FFF7FFFu) + 0x04000400u);
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(df_short2, m), u));
}
__device__ __forceinline__ uint32_t unbias_f16x2(uint32_t m) {
    const int hi = (int)(int16_t)(m >> 16), lo = (int)(int16_t)(m & 0xFFFFu);
    return __float_as_uint(f16_to_f32((uint32_t)max(max(hi, lo) - 0x400, 0)));
}

// ------------------------------------------------------------- host side --
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();
int launch_status(const char* what);  // DF_OK or DF_ERR_HIP (checks hipGetLastError)
int device_cu_count();                 // compute units of the current device (cached; 0 on error)
// One block folds `nparts` absmax partials (fold_* bit patterns) into
// absmax_out and/or the rule-D1/D2 scale for `fmt` (quant.hip).
void launch_absmax_fold(const uint32_t* partial, int nparts, int fmt, float* absmax_out, float* scale_out,
                        hipStream_t st);

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
inline bool aligned128(const void* p) { return ((uintptr_t)p & 127u) == 0; }
inline bool aligned4(const void* p) { return ((uintptr_t)p & 3u) == 0; }
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace dfk

#define DF_CHECK(cond, code, ...)          \
    do {                                   \
        if (!(cond)) {                     \
            ::dfk::set_error(__VA_ARGS__); \
            return (code);                 \
        }                                  \
    } while (0)
