/*
 * df_oracle.c -- CPU restatement of the fp8 Linear path (TEST INFRASTRUCTURE).
 * The contract it pins (D1-D5) and what checks each function is listed in
 * df_oracle.h.  Build: oracle/Makefile (gcc -O2, no -ffast-math, so binary32
 * division, multiplication and the sequential FC sums are IEEE round-to-nearest
 * and keep the reference's summation order).
 */
#include "df_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* OCP OFP8 v1.0 format parameters                                          */
/* ------------------------------------------------------------------------ */
typedef struct {
    int mbits;          /* mantissa (trailing significand) bits */
    int bias;           /* exponent bias */
    uint32_t max_bits;  /* binary32 bit pattern of the largest finite value */
    uint8_t max_code;   /* code of the largest finite value */
} fp8_fmt;

static const fp8_fmt FMTS[2] = {
    /* e4m3: S.EEEE.MMM, bias 7, max 1.75*2^8 = 448, NaN S.1111.111, no inf */
    {3, 7, 0x43E00000u, 0x7E},
    /* e5m2: S.EEEEE.MM, bias 15, max 1.75*2^15 = 57344, inf S.11111.00 */
    {2, 15, 0x47600000u, 0x7B},
};

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float dfo_fmax(int fmt) { return u2f(FMTS[fmt & 1].max_bits); }

/* Encode binary32 -> fp8, round to nearest even, saturating (D3).
 * Normal targets: re-bias the binary32 exponent and round the significand in
 * the integer domain (a carry out of the significand moves into the
 * exponent, which is the correct next binade).  Subnormal targets: the value
 * times 2^(bias-1+mbits) is exact, and rounding it to an integer with the
 * default (nearest-even) mode gives the subnormal code directly. */
uint8_t dfo_encode(float v, int fmt) {
    const fp8_fmt* f = &FMTS[fmt & 1];
    uint32_t u = f2u(v);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return sign | 0x7F;          /* NaN */
    if (a >= f->max_bits) return sign | f->max_code;  /* >= max, incl. inf */
    int e = (int)(a >> 23);
    int et = e - 127 + f->bias;                       /* fp8 biased exponent */
    if (et >= 1) {
        int sh = 23 - f->mbits;
        uint32_t r = a - ((uint32_t)(127 - f->bias) << 23);
        uint32_t lsb = (r >> sh) & 1u;
        r += ((1u << (sh - 1)) - 1u) + lsb;
        return sign | (uint8_t)(r >> sh);
    }
    float m = fabsf(v) * ldexpf(1.0f, f->bias - 1 + f->mbits);
    return sign | (uint8_t)(int)rintf(m);
}

float dfo_decode(uint8_t q, int fmt) {
    const fp8_fmt* f = &FMTS[fmt & 1];
    uint32_t sign = (uint32_t)(q & 0x80u) << 24;
    int ebits = 7 - f->mbits;
    int e = (q >> f->mbits) & ((1 << ebits) - 1);
    int m = q & ((1 << f->mbits) - 1);
    if (fmt == DFO_E4M3) {
        if ((q & 0x7F) == 0x7F) return u2f(sign | 0x7FC00000u);
    } else if (e == 31) {
        return m == 0 ? u2f(sign | 0x7F800000u) : u2f(sign | 0x7FC00000u);
    }
    float val;
    if (e == 0)
        val = ldexpf((float)m, 1 - f->bias - f->mbits);
    else
        val = ldexpf((float)((1 << f->mbits) + m), e - f->bias - f->mbits);
    return sign ? -val : val;
}

uint16_t dfo_f32_to_bf16(float v) {
    uint32_t u = f2u(v);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)(((u >> 16) & 0x8000u) | 0x7FC0u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float dfo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* binary32 -> IEEE binary16 (1 sign, 5 exponent bits of bias 15, 10 fraction
 * bits), round to nearest even.  |v| >= 65520 (the midpoint between the
 * largest finite 65504 and 2^16, which ties to the even 2^16) overflows to
 * inf; binary16 subnormals (|v| < 2^-14, unit 2^-24) are honoured; NaN gives
 * the quiet NaN sign|0x7E00 (the same policy as the bf16 rounding). */
uint16_t dfo_f32_to_f16(float v) {
    uint32_t u = f2u(v);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (a >= 0x38800000u) { /* 2^-14 and up: a normal binary16 */
        uint32_t r = a - ((uint32_t)(127 - 15) << 23);
        r = (r + 0x0FFFu + ((r >> 13) & 1u)) >> 13;
        return (uint16_t)(sign | r);
    }
    /* subnormal or zero: the value in units of 2^-24, rounded to an integer
     * (the scaling by a power of two is exact; 1024 is the smallest normal) */
    return (uint16_t)(sign | (uint16_t)rintf(u2f(a) * 0x1p24f));
}

/* IEEE binary16 -> binary32, exact; a NaN keeps its sign and payload (the
 * fraction shifted into the top of the binary32 fraction), like the bf16
 * widening. */
float dfo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 31) return u2f(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        float v = (float)m * 0x1p-24f; /* exact: m < 2^10 */
        return u2f(sign | f2u(v));
    }
    return u2f(sign | ((e - 15 + 127) << 23) | (m << 13));
}

/* ------------------------------------------------------------------------ */
/* Tensor operations                                                        */
/* ------------------------------------------------------------------------ */
float dfo_absmax_f32(const float* x, int64_t n) {
    float m = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        float a = fabsf(x[i]);
        if (isfinite(a) && a > m) m = a;
    }
    return m;
}

float dfo_absmax_bf16(const uint16_t* x, int64_t n) {
    float m = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        float a = fabsf(dfo_bf16_to_f32(x[i]));
        if (isfinite(a) && a > m) m = a;
    }
    return m;
}

float dfo_scale(float absmax, int fmt) {
    if (!(absmax > 0.0f) || !isfinite(absmax)) return 1.0f;
    float s = absmax / dfo_fmax(fmt);
    if (!(s > 0.0f) || !isfinite(s)) return 1.0f;
    return s;
}

void dfo_quantize_f32(const float* x, int64_t n, float s, int fmt, uint8_t* q) {
    for (int64_t i = 0; i < n; ++i) q[i] = dfo_encode(x[i] / s, fmt);
}

void dfo_quantize_bf16(const uint16_t* x, int64_t n, float s, int fmt, uint8_t* q) {
    for (int64_t i = 0; i < n; ++i) q[i] = dfo_encode(dfo_bf16_to_f32(x[i]) / s, fmt);
}

static inline float dequant_one(uint8_t q, float s, int fmt) {
    float d = dfo_decode(q, fmt);
    if (isnan(d)) return d; /* canonical quiet NaN with the code's sign */
    return d * s;
}

void dfo_dequantize_f32(const uint8_t* q, int64_t n, float s, int fmt, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = dequant_one(q[i], s, fmt);
}

void dfo_dequantize_bf16(const uint8_t* q, int64_t n, float s, int fmt, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = dfo_f32_to_bf16(dequant_one(q[i], s, fmt));
}

/* ------------------------------------------------------------------------ */
/* Threading helper: static split of [0, n) over nthreads pthreads          */
/* ------------------------------------------------------------------------ */
typedef void (*range_fn)(int64_t lo, int64_t hi, void* ctx, int tid);
typedef struct { range_fn fn; void* ctx; int64_t lo, hi; int tid; } range_job;

static void* range_thread(void* p) {
    range_job* j = (range_job*)p;
    j->fn(j->lo, j->hi, j->ctx, j->tid);
    return NULL;
}

static void parallel_range(int64_t n, int nthreads, range_fn fn, void* ctx) {
    if (nthreads <= 1 || n < 2) { fn(0, n, ctx, 0); return; }
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    range_job jobs[256];
    int64_t chunk = (n + nthreads - 1) / nthreads;
    int started = 0;
    for (int t = 0; t < nthreads; ++t) {
        int64_t lo = (int64_t)t * chunk, hi = lo + chunk;
        if (lo >= n) break;
        if (hi > n) hi = n;
        jobs[t] = (range_job){fn, ctx, lo, hi, t};
        if (pthread_create(&th[t], NULL, range_thread, &jobs[t]) != 0) {
            fn(lo, hi, ctx, t); /* run inline when a thread cannot start */
            th[t] = 0;
        }
        started = t + 1;
    }
    for (int t = 0; t < started; ++t)
        if (th[t]) pthread_join(th[t], NULL);
}

/* ------------------------------------------------------------------------ */
/* Exhaustive sweep helpers                                                 */
/* ------------------------------------------------------------------------ */
typedef struct { uint32_t first; int fmt; uint8_t* out; } enc_ctx;

static void enc_range(int64_t lo, int64_t hi, void* p, int tid) {
    (void)tid;
    enc_ctx* c = (enc_ctx*)p;
    for (int64_t i = lo; i < hi; ++i)
        c->out[i] = dfo_encode(u2f(c->first + (uint32_t)i), c->fmt);
}

void dfo_encode_bits_range(uint32_t first, int64_t count, int fmt, uint8_t* out, int nthreads) {
    enc_ctx c = {first, fmt, out};
    parallel_range(count, nthreads, enc_range, &c);
}

/* Elementwise conversion between the DType values 0 (binary32), 1
 * (binary16), 2 (int8) and 4 (bf16): widen to binary32 exactly, then round
 * once to the output type.  Returns 0, or -1 for a pair it does not
 * convert (the product's df_convert refuses the same pairs). */
static float widen(int dt, const void* in, int64_t i) {
    switch (dt) {
        case 0: return ((const float*)in)[i];
        case 1: return dfo_f16_to_f32(((const uint16_t*)in)[i]);
        case 2: return (float)((const int8_t*)in)[i];
        default: return dfo_bf16_to_f32(((const uint16_t*)in)[i]);
    }
}

int dfo_convert(int in_dtype, const void* in, int out_dtype, void* out, int64_t n) {
    const int in_ok = in_dtype == 0 || in_dtype == 1 || in_dtype == 2 || in_dtype == 4;
    const int out_ok = out_dtype == 0 || out_dtype == 1 || out_dtype == 4;
    if (!in_ok || !out_ok) return -1;
    for (int64_t i = 0; i < n; ++i) {
        float v = widen(in_dtype, in, i);
        if (out_dtype == 0) ((float*)out)[i] = v;
        else if (out_dtype == 1) ((uint16_t*)out)[i] = dfo_f32_to_f16(v);
        else ((uint16_t*)out)[i] = dfo_f32_to_bf16(v);
    }
    return 0;
}

/* Narrowing of every fp32 bit pattern in [first, first+count): bf16 (RNE) or
 * binary16 (RNE), the exhaustive-sweep helper of the conversion tests. */
typedef struct { uint32_t first; int to_f16; uint16_t* out; } narrow_ctx;

static void narrow_range(int64_t lo, int64_t hi, void* p, int tid) {
    (void)tid;
    narrow_ctx* c = (narrow_ctx*)p;
    if (c->to_f16)
        for (int64_t i = lo; i < hi; ++i) c->out[i] = dfo_f32_to_f16(u2f(c->first + (uint32_t)i));
    else
        for (int64_t i = lo; i < hi; ++i) c->out[i] = dfo_f32_to_bf16(u2f(c->first + (uint32_t)i));
}

void dfo_narrow_bits_range(uint32_t first, int64_t count, int to_f16, uint16_t* out, int nthreads) {
    narrow_ctx c = {first, to_f16, out};
    parallel_range(count, nthreads, narrow_range, &c);
}

/* Sorted values of the non-negative finite codes 0..max_code, built from the
 * spec's closed form (value = 2^(e-bias) * (1 + m/2^mbits), or
 * 2^(1-bias) * m/2^mbits when e == 0) in double precision. */
static double code_table[2][128];
static int code_table_len[2];
static pthread_once_t table_once = PTHREAD_ONCE_INIT;

static void build_tables(void) {
    for (int fmt = 0; fmt < 2; ++fmt) {
        const fp8_fmt* f = &FMTS[fmt];
        int n = f->max_code + 1;
        for (int c = 0; c < n; ++c) {
            int e = c >> f->mbits, m = c & ((1 << f->mbits) - 1);
            double frac = (double)m / (double)(1 << f->mbits);
            code_table[fmt][c] = e == 0 ? ldexp(frac, 1 - f->bias) : ldexp(1.0 + frac, e - f->bias);
        }
        code_table_len[fmt] = n;
    }
}

uint8_t dfo_encode_by_table(float v, int fmt) {
    pthread_once(&table_once, build_tables);
    fmt &= 1;
    uint8_t sign = signbit(v) ? 0x80 : 0x00;
    if (isnan(v)) return sign | 0x7F;
    double a = fabs((double)v);
    const double* t = code_table[fmt];
    int n = code_table_len[fmt];
    if (a >= t[n - 1]) return sign | (uint8_t)(n - 1);
    int lo = 0, hi = n - 1; /* invariant: t[lo] <= a < t[hi] */
    while (hi - lo > 1) {
        int mid = (lo + hi) / 2;
        if (t[mid] <= a) lo = mid; else hi = mid;
    }
    double dlo = a - t[lo], dhi = t[hi] - a;
    int c;
    if (dlo < dhi) c = lo;
    else if (dhi < dlo) c = hi;
    else c = (lo & 1) ? hi : lo;
    return sign | (uint8_t)c;
}

typedef struct { uint32_t first; int fmt; int64_t bad[256]; uint32_t first_bad[256]; } sweep_ctx;

static void sweep_range(int64_t lo, int64_t hi, void* p, int tid) {
    sweep_ctx* c = (sweep_ctx*)p;
    int64_t bad = 0;
    uint32_t fb = 0;
    for (int64_t i = lo; i < hi; ++i) {
        float v = u2f(c->first + (uint32_t)i);
        if (dfo_encode(v, c->fmt) != dfo_encode_by_table(v, c->fmt)) {
            if (bad == 0) fb = c->first + (uint32_t)i;
            ++bad;
        }
    }
    c->bad[tid] = bad;
    c->first_bad[tid] = fb;
}

int64_t dfo_sweep_compare(uint32_t first, int64_t count, int fmt, uint32_t* first_bad, int nthreads) {
    pthread_once(&table_once, build_tables);
    sweep_ctx* c = (sweep_ctx*)calloc(1, sizeof(sweep_ctx));
    if (!c) return -1;
    c->first = first;
    c->fmt = fmt & 1;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    parallel_range(count, nthreads, sweep_range, c);
    int64_t total = 0;
    int have = 0;
    for (int t = 0; t < nthreads; ++t) {
        if (c->bad[t] && !have && first_bad) { *first_bad = c->first_bad[t]; have = 1; }
        total += c->bad[t];
    }
    free(c);
    return total;
}

/* ------------------------------------------------------------------------ */
/* FC loops, restated from dnn/layers/fully_connected_layer.cu              */
/* ------------------------------------------------------------------------ */
typedef struct {
    const float *a, *b, *bias;
    float* out;
    int N, in_f, out_f;
} fc_ctx;

/* forward, :29-35 -- one row of tokens per work item */
static void fwd_rows(int64_t lo, int64_t hi, void* p, int tid) {
    (void)tid;
    fc_ctx* c = (fc_ctx*)p;
    for (int64_t n = lo; n < hi; ++n)
        for (int o = 0; o < c->out_f; ++o) {
            float sum = 0.f;
            const float* x = c->a + n * (int64_t)c->in_f;
            const float* w = c->b + (int64_t)o * c->in_f;
            for (int i = 0; i < c->in_f; ++i) sum += x[i] * w[i];
            sum += c->bias ? c->bias[o] : 0.f;
            c->out[n * (int64_t)c->out_f + o] = sum;
        }
}

void dfo_fc_forward(const float* X, const float* W, const float* b, float* Y,
                    int N, int in_f, int out_f, int nthreads) {
    fc_ctx c = {X, W, b, Y, N, in_f, out_f};
    parallel_range(N, nthreads, fwd_rows, &c);
}

/* GTest host oracle, tests/layers/fully_connected_layer_test.cu:38-43:
 * output starts at the bias, then accumulates. */
static void fwd_rows_bias_first(int64_t lo, int64_t hi, void* p, int tid) {
    (void)tid;
    fc_ctx* c = (fc_ctx*)p;
    for (int64_t n = lo; n < hi; ++n)
        for (int o = 0; o < c->out_f; ++o) {
            float acc = c->bias ? c->bias[o] : 0.f;
            const float* x = c->a + n * (int64_t)c->in_f;
            const float* w = c->b + (int64_t)o * c->in_f;
            for (int i = 0; i < c->in_f; ++i) acc += x[i] * w[i];
            c->out[n * (int64_t)c->out_f + o] = acc;
        }
}

void dfo_fc_forward_bias_first(const float* X, const float* W, const float* b, float* Y,
                               int N, int in_f, int out_f, int nthreads) {
    fc_ctx c = {X, W, b, Y, N, in_f, out_f};
    parallel_range(N, nthreads, fwd_rows_bias_first, &c);
}

/* dX, :54-59 -- dX[n,i] = sum_j dY[n,j] * W[j,i], j sequential */
static void bwd_in_rows(int64_t lo, int64_t hi, void* p, int tid) {
    (void)tid;
    fc_ctx* c = (fc_ctx*)p;
    for (int64_t n = lo; n < hi; ++n)
        for (int i = 0; i < c->in_f; ++i) {
            float sum = 0.f;
            const float* dy = c->a + n * (int64_t)c->out_f;
            for (int j = 0; j < c->out_f; ++j) sum += dy[j] * c->b[(int64_t)j * c->in_f + i];
            c->out[n * (int64_t)c->in_f + i] = sum;
        }
}

void dfo_fc_backward_input(const float* dY, const float* W, float* dX,
                           int N, int in_f, int out_f, int nthreads) {
    fc_ctx c = {dY, W, NULL, dX, N, in_f, out_f};
    parallel_range(N, nthreads, bwd_in_rows, &c);
}

/* dW, :78-87 -- dW[o,i] = sum_n dY[n,o] * X[n,i], n sequential, overwrite */
static void bwd_w_rows(int64_t lo, int64_t hi, void* p, int tid) {
    (void)tid;
    fc_ctx* c = (fc_ctx*)p;
    for (int64_t o = lo; o < hi; ++o)
        for (int i = 0; i < c->in_f; ++i) {
            float sum = 0.f;
            for (int n = 0; n < c->N; ++n)
                sum += c->a[(int64_t)n * c->out_f + o] * c->b[(int64_t)n * c->in_f + i];
            c->out[o * (int64_t)c->in_f + i] = sum;
        }
}

void dfo_fc_backward_weights(const float* dY, const float* X, float* dW,
                             int N, int in_f, int out_f, int nthreads) {
    fc_ctx c = {dY, X, NULL, dW, N, in_f, out_f};
    parallel_range(out_f, nthreads, bwd_w_rows, &c);
}

/* db, :99-105 -- db[o] = sum_n dY[n,o], n sequential */
void dfo_fc_backward_bias(const float* dY, float* db, int N, int out_f) {
    for (int o = 0; o < out_f; ++o) {
        float sum = 0.f;
        for (int n = 0; n < N; ++n) sum += dY[(int64_t)n * out_f + o];
        db[o] = sum;
    }
}

/* ------------------------------------------------------------------------ */
/* Consumer side: global-norm clipping and Adam                             */
/* ------------------------------------------------------------------------ */

/* Sum of RN32(x*x) in binary64, sequential. */
double dfo_sumsq(const float* x, int64_t n) {
    double s = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        const float q = x[i] * x[i];
        s += (double)q;
    }
    return s;
}

/* Product contract: squares in binary32 (clip_grad_norm.cu:41-43 forms them
 * that way), accumulated in binary64, root rounded once to binary32. */
float dfo_grad_norm(const float* const* g, const int64_t* n, int count) {
    double s = 0.0;
    for (int t = 0; t < count; ++t) s += dfo_sumsq(g[t], n[t]);
    return (float)sqrt(s);
}

/* The reference's own host norm, clip_grad_norm.cu:36-50: a binary32
 * running sum per tensor, binary32 total, sqrt in binary32. */
float dfo_grad_norm_ref_f32(const float* const* g, const int64_t* n, int count) {
    float total = 0.0f;
    for (int t = 0; t < count; ++t) {
        float sum_sq = 0.0f;
        for (int64_t i = 0; i < n[t]; ++i) sum_sq += g[t][i] * g[t][i];
        total += sum_sq;
    }
    return sqrtf(total);
}

/* clip_grad_norm.cu:18 (kernel) and :55 (condition): grad * (max_norm / norm)
 * when norm > max_norm.  Returns 1 when it scaled. */
int dfo_clip_scale(float* g, int64_t n, float norm, float max_norm) {
    if (!(norm > max_norm)) return 0;
    const float f = max_norm / norm;
    for (int64_t i = 0; i < n; ++i) g[i] = g[i] * f;
    return 1;
}

/* 1 - beta^t: beta^t rounded once to binary32, then the binary32
 * subtraction (adam_optimizer.cu:28-29 writes T(1.0) - pow(beta, t)). */
float dfo_bias_correction(float beta, int t) {
    return 1.0f - (float)pow((double)beta, (double)t);
}

/* adam_optimizer.cu:24-30 (float path), element by element, each binary32
 * operation rounded in the order written; `clip_factor` multiplies the
 * gradient first (1.0f leaves it unchanged). */
void dfo_adam_step(float* p, const float* grad, float* m, float* v, int64_t n,
                   float lr, float beta1, float beta2, float eps, float wd, int t,
                   float clip_factor) {
    const float bc1 = dfo_bias_correction(beta1, t);
    const float bc2 = dfo_bias_correction(beta2, t);
    const float omb1 = 1.0f - beta1, omb2 = 1.0f - beta2;
    for (int64_t i = 0; i < n; ++i) {
        const float gr = grad[i] * clip_factor;
        const float g = gr + wd * p[i];
        m[i] = beta1 * m[i] + omb1 * g;
        v[i] = beta2 * v[i] + omb2 * g * g;
        const float m_hat = m[i] / bc1;
        const float v_hat = v[i] / bc2;
        p[i] = p[i] - lr * m_hat / (sqrtf(v_hat) + eps);
    }
}

/* ------------------------------------------------------------------------ */
/* Delayed scaling: amax history                                            */
/* ------------------------------------------------------------------------ */

/* Push `amax` as the newest entry (history[0]); the others move up one and
 * the oldest drops out.  Returns the scale (D1/D2) of the new history's
 * maximum: the scale the next pass uses. */
float dfo_history_push(float* history, int len, float amax, int fmt) {
    for (int i = len - 1; i > 0; --i) history[i] = history[i - 1];
    history[0] = amax;
    float m = 0.0f;
    for (int i = 0; i < len; ++i) m = history[i] > m ? history[i] : m;
    return dfo_scale(m, fmt);
}

/* ------------------------------------------------------------------------ */
/* LayerNorm (dnn/layers/layer_norm_layer.cu:26-63)                          */
/* ------------------------------------------------------------------------ */

/* One row per iteration, as the reference's thread 0 does: sequential
 * binary32 sum for the mean, sequential sum of squared deviations (the
 * product-add as one fused multiply-add, the contraction nvcc applies by
 * default), var = sum / C, rstd = 1 / sqrt(var + eps) (correctly rounded
 * steps; the reference's rsqrtf is an approximation within 2 ulp), then
 * y = (x - mean) * rstd and, with gamma/beta, fma(y, gamma, beta) (again the
 * default contraction of `norm * gamma + beta`).  round_bf16 != 0 rounds y
 * to bf16 (RNE), the reference's cast to T for a bf16 tensor. */
void dfo_layernorm(const float* x, int rows, int C, const float* gamma, const float* beta,
                   float eps, int round_bf16, float* y) {
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (int64_t)r * C;
        float sum = 0.0f;
        for (int i = 0; i < C; ++i) sum += xr[i];
        const float mean = sum / (float)C;
        float sq = 0.0f;
        for (int i = 0; i < C; ++i) {
            const float d = xr[i] - mean;
            sq = fmaf(d, d, sq);
        }
        const float var = sq / (float)C;
        const float rstd = 1.0f / sqrtf(var + eps);
        for (int i = 0; i < C; ++i) {
            float n = (xr[i] - mean) * rstd;
            if (gamma) n = fmaf(n, gamma[i], beta[i]);
            y[(int64_t)r * C + i] = round_bf16 ? dfo_bf16_to_f32(dfo_f32_to_bf16(n)) : n;
        }
    }
}
