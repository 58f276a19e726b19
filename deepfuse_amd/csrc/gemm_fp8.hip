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
// Main kernel (gemm_nt_dma128_kernel): a block of WM x WN waves owns a
// BM x BN tile of C (256x256 with 8 waves of 128x64, two waves per SIMD, for
// large outputs); each wave owns (BM/WM) x (BN/WN) as 32x32
// v_mfma_f32_32x32x64_f8f6f4 tiles with fp32 accumulators.  Operand tiles
// move global -> LDS by buffer_load_dwordx4 ... lds (no VGPR staging), K
// advancing 128 bytes per step through two LDS stages: the DMA for step k+1
// runs under the MFMAs of step k, one barrier per step.  The epilogue stages
// results through LDS so stores are whole row segments.  A register-staged
// kernel (gemm_nt_kernel) covers operands whose byte range does not fit a
// 32-bit buffer resource.
//
// Tile order: blocks are dispatched round-robin over the 8 XCDs; the block
// id is remapped so each XCD owns a contiguous range of tiles, walked in
// groups of GROUP_M tile-rows so neighbouring blocks share A and B in their
// XCD's L2.
//
// Split-K (small outputs with long reductions, e.g. dW): grid.y = S slices
// of the K range write raw fp32 partial tiles to a workspace; a reduce pass
// sums them in slice order (deterministic) and applies scale, bias and the
// output conversion.
//
// Replaces the reference's fully_connected_forward_kernel, fc_backward_input
// and fc_backward_weights (dnn/layers/fully_connected_layer.cu:14-89).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "df_common.hpp"
#include "gemm_sched.hpp"

namespace dfk {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kBK = 128;              // bytes of K per step = one MFMA depth
constexpr int kLdsStride = kBK + 16;  // padded LDS row (bytes)
constexpr int kGroupM = 8;

template <typename T> struct OutCvt;
template <> struct OutCvt<float> {
    static __device__ __forceinline__ float cvt(float v) { return v; }
};
template <> struct OutCvt<uint16_t> {  // bf16 bits
    static __device__ __forceinline__ uint16_t cvt(float v) { return (uint16_t)f32_to_bf16_rne(v); }
};
template <> struct OutCvt<f16_t> {
    static __device__ __forceinline__ f16_t cvt(float v) { return f16_t{(uint16_t)f32_to_f16_rne(v)}; }
};
__device__ __forceinline__ float bias_ld(const float* b, int i) { return b[i]; }
__device__ __forceinline__ float bias_ld(const uint16_t* b, int i) { return bf16_to_f32(b[i]); }
__device__ __forceinline__ float bias_ld(const f16_t* b, int i) { return f16_to_f32(b[i].bits); }

// 4 consecutive outputs of one row: one 16-byte (fp32) or 8-byte (bf16) store
__device__ __forceinline__ void store4(float* p, const float* v) {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
}
__device__ __forceinline__ void store4(uint16_t* p, const float* v) {
    *reinterpret_cast<u32x2*>(p) = u32x2{f32_to_bf16_rne(v[0]) | (f32_to_bf16_rne(v[1]) << 16),
                                        f32_to_bf16_rne(v[2]) | (f32_to_bf16_rne(v[3]) << 16)};
}
__device__ __forceinline__ void store4(f16_t* p, const float* v) {
    *reinterpret_cast<u32x2*>(p) = u32x2{f32_to_f16_rne(v[0]) | (f32_to_f16_rne(v[1]) << 16),
                                        f32_to_f16_rne(v[2]) | (f32_to_f16_rne(v[3]) << 16)};
}

__device__ __forceinline__ v8i lds_frag(const uint8_t* p) {
    const u32x4 lo = *reinterpret_cast<const u32x4*>(p);
    const u32x4 hi = *reinterpret_cast<const u32x4*>(p + 16);
    v8i r;
    r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
    r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
    return r;
}

// logical tile (tm, tn) of block `pid` in a grid of tiles_m x tiles_n
__device__ __forceinline__ void tile_of(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int nblk = tiles_m * tiles_n;
    const int q = nblk >> 3, r = nblk & 7;
    const int xcd = pid & 7, idx = pid >> 3;
    const int logical = xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
    const int per_group = kGroupM * tiles_n;
    const int group = logical / per_group;
    const int first_m = group * kGroupM;
    const int gsize = min(tiles_m - first_m, kGroupM);
    const int in_group = logical - group * per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

template <int BM, int BN, int WM, int WN, int FA, int FB, typename OutT, typename BiasT, bool SPLIT>
__global__ __launch_bounds__(64 * WM * WN, 1) void gemm_nt_kernel(
    const uint8_t* __restrict__ A, int lda, const uint8_t* __restrict__ B, int ldb, int M, int N,
    int K, int k_per_split, const float* __restrict__ sa, const float* __restrict__ sb,
    const BiasT* __restrict__ bias, OutT* __restrict__ C, int ldc, bool vec_out,
    float* __restrict__ partial) {
    constexpr int NT = 64 * WM * WN;
    constexpr int TM = BM / WM, TN = BN / WN;  // wave tile
    constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 MFMA tiles per wave
    constexpr int CA = BM * (kBK / 16) / NT;   // 16-byte chunks per thread per step
    constexpr int CB = BN * (kBK / 16) / NT;
    static_assert(CA * NT == BM * (kBK / 16) && CB * NT == BN * (kBK / 16), "tile/threads mismatch");
    static_assert(FM * 32 == TM && FN * 32 == TN, "wave tile must be a multiple of 32");
    __shared__ __attribute__((aligned(16))) uint8_t sA[2][BM * kLdsStride];
    __shared__ __attribute__((aligned(16))) uint8_t sB[2][BN * kLdsStride];

    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int wm = w / WN, wn = w % WN;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int kbeg = SPLIT ? blockIdx.y * k_per_split : 0;
    const int kend = SPLIT ? min(K, kbeg + k_per_split) : K;

    // chunk c of a tile: row c/8, byte column (c%8)*16; thread t owns c = t + NT*i
    u32x4 ra[CA], rb[CB];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int c = t + NT * i;
            const int r = c >> 3, gk = k0 + (c & 7) * 16, gm = m0 + r;
            ra[i] = (gm < M && gk < kend) ? *reinterpret_cast<const u32x4*>(A + (int64_t)gm * lda + gk)
                                          : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int c = t + NT * i;
            const int r = c >> 3, gk = k0 + (c & 7) * 16, gn = n0 + r;
            rb[i] = (gn < N && gk < kend) ? *reinterpret_cast<const u32x4*>(B + (int64_t)gn * ldb + gk)
                                          : u32x4{0, 0, 0, 0};
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int c = t + NT * i;
            *reinterpret_cast<u32x4*>(&sA[buf][(c >> 3) * kLdsStride + (c & 7) * 16]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int c = t + NT * i;
            *reinterpret_cast<u32x4*>(&sB[buf][(c >> 3) * kLdsStride + (c & 7) * 16]) = rb[i];
        }
    };

    v16f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int nk = kend > kbeg ? (kend - kbeg + kBK - 1) / kBK : 0;
    if (nk > 0) {
        gload(kbeg);
        lstore(0);
    }
    __syncthreads();

    // MFMA operand layout (32x32x64, 8-bit): lane l supplies row l%32 of its
    // operand and 32 bytes of K at byte offset 32*(l/32); A and B share the
    // layout.  The B fragment goes in the instruction's first operand slot,
    // so the 32x32 accumulator is C^T: lane l holds row l%32 of C, and
    // register 4*g + i holds column 8*g + 4*(l/32) + i -- four runs of four
    // consecutive columns, each stored as one vector.
    const int fr = lane & 31, fk = (lane >> 5) * 32;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload(kbeg + (kt + 1) * kBK);
        const uint8_t* pa = &sA[cur][(wm * TM + fr) * kLdsStride + fk];
        const uint8_t* pb = &sB[cur][(wn * TN + fr) * kLdsStride + fk];
#pragma unroll
        for (int kc = 0; kc < kBK; kc += 64) {
            v8i bfr[FN];
#pragma unroll
            for (int j = 0; j < FN; ++j) bfr[j] = lds_frag(pb + j * 32 * kLdsStride + kc);
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const v8i afr = lds_frag(pa + i * 32 * kLdsStride + kc);
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bfr[j], afr, acc[i][j], FB, FA,
                                                                                0, 0, 0, 0);
            }
        }
        if (kt + 1 < nk) lstore(cur ^ 1);
        __syncthreads();
    }

    const int hi = (lane >> 5) * 4;
    if (SPLIT) {
        float* P = partial + (int64_t)blockIdx.y * M * N;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int row = m0 + wm * TM + i * 32 + fr;
            if (row >= M) continue;
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int col = n0 + wn * TN + j * 32 + 8 * g + hi;
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (col + r < N) P[(int64_t)row * N + col + r] = acc[i][j][4 * g + r];
                }
        }
        return;
    }
    const float sab = sa[0] * sb[0];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int row = m0 + wm * TM + i * 32 + fr;
        if (row >= M) continue;
        OutT* crow = C + (int64_t)row * ldc;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int col = n0 + wn * TN + j * 32 + 8 * g + hi;
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    v[r] = acc[i][j][4 * g + r] * sab + ((bias && col + r < N) ? bias_ld(bias, col + r) : 0.0f);
                if (vec_out && col + 3 < N) {
                    store4(crow + col, v);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (col + r < N) crow[col + r] = OutCvt<OutT>::cvt(v[r]);
                }
            }
    }
}

// Wave-private LDS staging of a (TM x TN) accumulator tile held in the
// C^T layout of 32x32 MFMA tiles (lane l: row l%32, register 4g+i = column
// 8g + 4(l/32) + i).  Values are scaled, biased and converted in registers,
// written to a padded [32][TN] slab per 32-row group, then read back row
// contiguous: 16 bytes per lane, whole row segments per store instruction.
template <typename OutT, int TM, int TN, int FM, int FN, typename BiasT>
__device__ __forceinline__ void epilogue_lds(const v16f (&acc)[FM][FN], uint8_t* lds, int w, int lane,
                                             int row0, int col0, int M, int N, OutT* __restrict__ C,
                                             int ldc, bool vec_ok, float scale,
                                             const BiasT* __restrict__ bias) {
    constexpr int ES = (int)sizeof(OutT);
    constexpr int ROWB = TN * ES + 16;   // padded slab row (bytes)
    constexpr int SLAB = 32 * ROWB;
    constexpr int CPR = TN * ES / 16;    // 16-byte chunks per slab row
    constexpr int EPC = 16 / ES;         // elements per chunk
    static_assert(CPR * 16 == TN * ES && 64 % CPR == 0, "slab row must split into 16-byte chunks");
    constexpr int RPI = 64 / CPR;        // rows per store instruction
    uint8_t* slab = lds + w * SLAB;
    const int fr = lane & 31, hi = (lane >> 5) * 4;
    float bv[FN][4][4];
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int col = col0 + j * 32 + 8 * g + hi + r;
                bv[j][g][r] = (bias && col < N) ? bias_ld(bias, col) : 0.0f;
            }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = acc[i][j][4 * g + r] * scale + bv[j][g][r];
                store4(reinterpret_cast<OutT*>(slab + fr * ROWB + (j * 32 + 8 * g + hi) * ES), v);
            }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): slab written
#pragma unroll
        for (int q = 0; q < 32 / RPI; ++q) {
            const int rr = q * RPI + lane / CPR;
            const int cc = (lane % CPR) * EPC;
            const u32x4 val = *reinterpret_cast<const u32x4*>(slab + rr * ROWB + cc * ES);
            const int row = row0 + i * 32 + rr, col = col0 + cc;
            if (row < M) {
                OutT* dst = C + (int64_t)row * ldc + col;
                if (vec_ok && col + EPC <= N) {
                    *reinterpret_cast<u32x4*>(dst) = val;
                } else {
                    const OutT* e = reinterpret_cast<const OutT*>(&val);
#pragma unroll
                    for (int x = 0; x < EPC; ++x)
                        if (col + x < N) dst[x] = e[x];
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // slab read before the next rows overwrite it
    }
}

// ---------------------------------------------------------------------------
// Full-line LDS-DMA variant: K advances 128 bytes per step (whole 128-byte
// cache lines per row; each DMA instruction fills 8 rows x 128 bytes) through
// two LDS stages.  Chunk c of row r sits in slot c ^ g(r),
// g(r) = ((r >> 1) ^ (r >> 4)) & 7, which keeps the 16 or 32 rows of one
// ds_read_b128 pass in distinct bank groups.  Within a step the fragments of
// the second K=64 half are read while the first half's MFMAs run.
__device__ __forceinline__ int swz128(int r) { return ((r >> 1) ^ (r >> 4)) & 7; }

template <int BM, int BN, int WM, int WN, int FA, int FB, typename OutT, typename BiasT, bool SPLIT>
__global__ __launch_bounds__(64 * WM * WN, 1) void gemm_nt_dma128_kernel(
    const uint8_t* __restrict__ A, int lda, const uint8_t* __restrict__ B, int ldb, int M, int N,
    int K, int k_per_split, const float* __restrict__ sa, const float* __restrict__ sb,
    const BiasT* __restrict__ bias, OutT* __restrict__ C, int ldc, bool vec_out,
    float* __restrict__ partial) {
    constexpr int NW = WM * WN;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int IA = BM / 8 / NW, IB = BN / 8 / NW;  // DMA instructions per wave per step
    static_assert(IA * NW * 8 == BM && IB * NW * 8 == BN, "rows must split evenly over waves");
    static_assert(FM * 32 == TM && FN * 32 == TN, "wave tile must be a multiple of 32");
    constexpr int STAGE = (BM + BN) * kBK;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * STAGE];

    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int wm = w / WN, wn = w % WN;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int kbeg = SPLIT ? blockIdx.y * k_per_split : 0;
    const int kend = SPLIT ? min(K, kbeg + k_per_split) : K;

    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, M * lda, 0x00020000);
    const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, N * ldb, 0x00020000);
    constexpr uint32_t kOOB = 0x80000000u;
    const int drow = lane >> 3, dslot = lane & 7;
    auto dma = [&](int step, int stage) {
        uint8_t* base = lds + stage * STAGE;
        const int k0 = kbeg + step * kBK;
#pragma unroll
        for (int i = 0; i < IA; ++i) {
            const int r = (w * IA + i) * 8 + drow;
            const int gk = k0 + ((dslot ^ swz128(r)) << 4);
            const int gm = m0 + r;
            const uint32_t off = (gk < kend && gm < M) ? (uint32_t)(gm * lda + gk) : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rA, (__attribute__((address_space(3))) void*)(base + (w * IA + i) * 8 * kBK), 16, off, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < IB; ++i) {
            const int r = (w * IB + i) * 8 + drow;
            const int gk = k0 + ((dslot ^ swz128(r)) << 4);
            const int gn = n0 + r;
            const uint32_t off = (gk < kend && gn < N) ? (uint32_t)(gn * ldb + gk) : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rB, (__attribute__((address_space(3))) void*)(base + BM * kBK + (w * IB + i) * 8 * kBK), 16, off,
                0, 0, 0);
        }
    };

    v16f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int fr = lane & 31, fh = (lane >> 5) * 2;
    auto frag = [&](const uint8_t* stage_rows, int row, int kc) {
        const int s0 = ((kc >> 4) + fh) ^ swz128(row);
        const uint8_t* p = stage_rows + row * kBK;
        const u32x4 lo = *reinterpret_cast<const u32x4*>(p + s0 * 16);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(p + (s0 ^ 1) * 16);
        v8i r;
        r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
        r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
        return r;
    };
    auto load_frags = [&](int stage, int kc, v8i* af, v8i* bf) {
        const uint8_t* sa_ = lds + stage * STAGE;
        const uint8_t* sb_ = sa_ + BM * kBK;
#pragma unroll
        for (int j = 0; j < FN; ++j) bf[j] = frag(sb_, wn * TN + j * 32 + fr, kc);
#pragma unroll
        for (int i = 0; i < FM; ++i) af[i] = frag(sa_, wm * TM + i * 32 + fr, kc);
    };
    auto mma = [&](const v8i* af, const v8i* bf) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[j], af[i], acc[i][j], FB, FA,
                                                                            0, 0, 0, 0);
    };

    const int nk = kend > kbeg ? (kend - kbeg + kBK - 1) / kBK : 0;
    if (nk > 0) dma(0, 0);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __builtin_amdgcn_s_barrier();
    v8i a0[FM], b0[FN], a1[FM], b1[FN];
    for (int k = 0; k < nk; ++k) {
        const int cur = k & 1;
        load_frags(cur, 0, a0, b0);
        if (k + 1 < nk) dma(k + 1, cur ^ 1);
        load_frags(cur, 64, a1, b1);
        mma(a0, b0);
        mma(a1, b1);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): next stage landed
        __builtin_amdgcn_s_barrier();
    }

    if (SPLIT)
        epilogue_lds<float, TM, TN, FM, FN>(acc, lds, w, lane, m0 + wm * TM, n0 + wn * TN, M, N,
                                            partial + (int64_t)blockIdx.y * M * N, N, (N & 3) == 0,
                                            1.0f, (const BiasT*)nullptr);
    else
        epilogue_lds<OutT, TM, TN, FM, FN>(acc, lds, w, lane, m0 + wm * TM, n0 + wn * TN, M, N, C, ldc,
                                           vec_out, sa[0] * sb[0], bias);
}

// ---------------------------------------------------------------------------
// Persistent kernel for outputs with at least one 256x256 tile per CU.
//
// One block per CU (grid = min(tiles, CUs)) walks tiles bl, bl+P, bl+2P, ...
// of the grouped tile order; bl remaps the block id so that each XCD owns a
// contiguous range of P/8 concurrent tiles (sharing A rows and B columns in
// its L2).  8 waves, two per SIMD, each owning a 128x64 quarter-row of the
// 256x256 tile as 4x2 v_mfma_f32_32x32x64_f8f6f4 tiles (narrow tiles:
// 256x128, a 64x64 part per wave as 2x2 MFMA tiles).
//
// Pipeline: K advances in half-steps of 64 bytes (one MFMA depth).  A DMA
// step moves 128 bytes of K (whole cache lines) for the tile's 256 A rows
// and 256 B rows into one of two 64 KiB LDS stages.  Half-step h issues the
// MFMAs on fragments h and reads fragments h+1 from LDS.  At the start of
// each odd half-step 2g+1 a wave waits for its part of DMA step g+1, the
// block synchronises, and DMA step g+2 goes into stage g%2, whose last reads
// were in half-step 2g.  The DMA cursor runs across tile boundaries, so the
// next tile's first steps load while this tile finishes and stores.
//
// LDS rows are 128 bytes; 16-byte chunk c of row r sits in slot
// c ^ ((r >> 1) & 7), which spreads the 16 rows read by each group of 16
// lanes over all 64 banks (no bank conflicts for the fragment reads).
//
// Bias: every DMA step also moves the tile's bias slice (4 bytes per lane)
// into one of three 2 KiB LDS slots (tile index mod 3), so the epilogue reads
// it from LDS.  Epilogue: scale, bias and the bf16 conversion
// (v_cvt_pk_bf16_f32, round to nearest even) in registers, then each 32-row
// block passes through the wave's LDS slab and leaves as 16-byte stores, 8
// lanes per 128-byte row segment, non-temporal: the output streams past L2,
// leaving it to the operand panels (2-3% less step time at config 4 than
// plain stores).
constexpr int kPBM = 256, kPBN = 256;  // persistent block tile
constexpr int kPKB = 128;              // K bytes per DMA step
constexpr int kPStage = (kPBM + kPBN) * kPKB;
constexpr int kPBiasSlots = 3;
constexpr int kPBiasSlot = 2048;

typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16_rne(float a, float b) {
    const v2f f = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, v2bf));
}

// s_waitcnt immediate (gfx9 encoding): vmcnt(n), lgkmcnt(0), no expcnt wait
__device__ __forceinline__ constexpr int waitcnt_vm_lgkm0(int n) {
    return (n & 15) | ((n >> 4) << 14) | 0x70;
}

// The lane index, computed afresh where it is called.  The asm is opaque to
// the optimiser, so offsets derived from it stay where they are used: taken
// from threadIdx, the epilogue's per-lane offsets were hoisted out of the
// tile loop and, at the main loop's register pressure, spilled; each reload
// in the epilogue then waited on vmcnt(0), i.e. for the DMA in flight.
__device__ __forceinline__ int fresh_lane() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

// Epilogue geometry for an output element of ES bytes: each 32-row block of
// a wave's FMR*32 x 64 part passes through an LDS slab of SR rows.
template <int ES, int FMR = 4>
struct EpiGeom {
    static constexpr int SR = ES == 2 ? 16 : 8;          // slab rows
    static constexpr int SROW = 64 * ES + 16;            // padded slab row (bytes)
    static constexpr int SLAB = SR * SROW;
    static constexpr int NPASS = 32 / SR;                // slab passes per 32-row block
    static constexpr int SPP = SR * 64 * ES / 1024;      // 16-byte stores per lane per pass
    static constexpr int NST = FMR * NPASS * SPP;        // epilogue stores per wave
};

// The second GEMM of a grouped launch (see gemm_sched.hpp): its operands,
// output and scales; never split, no bias.
struct PProb {
    const uint8_t* A;
    const uint8_t* B;
    void* C;
    const float* sa;
    const float* sb;
    int lda, ldb, M, N, K, ldc, vec_out;  // vec_out: an epi_store_mode
};

// cost of a work unit beyond its DMA steps (pipeline fill, epilogue), in
// the steps of the grouped schedule
constexpr int kUnitOverhead = 3;

template <typename T> struct Tag { using type = T; };

// NARROW: 256x128 tiles (one problem, unsplit).  The eight waves own 64x64
// parts (4 x 2 waves, 2x2 MFMA tiles each); a DMA step moves the 256 A rows
// and 128 B rows, so each wave issues two B instructions instead of four.
// For outputs whose 256x256 tiles would leave CUs idle or a last round
// mostly empty (the plan below compares both).
// TIMELINE (a diagnostic instantiation, df_fp8_gemm_fwd_timeline): lane 0
// of wave 0 writes the 100 MHz real-time counter to tl[block][...] at the
// block's start ([0]) and, for its tile t, at the tile's first half-step
// ([1 + 3t]), before its epilogue ([2 + 3t]) and after it ([3 + 3t]), while
// 1 + 3t + 2 < tl_per_block; every other instantiation compiles none of it.
// AMAX_OUT (df_fp8_gemm_fwd_absmax: one problem, unsplit; df_fp8_gemm_bwd_absmax:
// grouped, the second problem's (dX's) tiles only; bf16 or fp32 output):
// the epilogue also folds |C| over the finite values it stores, as stored
// (after the conversion to the output type), with the compare-free biased
// folds, and after its last tile wave w of block bl writes its maximum (a
// binary32 pattern) to amax_part[bl * 8 + w].
template <int FA, int FB, typename OutT, typename BiasT, bool HAS_BIAS, bool SPLIT, typename OutT1, bool NARROW,
          bool TIMELINE = false, bool AMAX_OUT = false>
__device__ __forceinline__ void persistent_body(
    const uint8_t* __restrict__ A, int lda, const uint8_t* __restrict__ B, int ldb, int M, int N, int K,
    const float* __restrict__ sa, const float* __restrict__ sb, const BiasT* __restrict__ bias,
    OutT* __restrict__ C, int ldc, int vec_out, int ksteps, int nsplit, const PProb& p1,
    uint64_t* __restrict__ tl = nullptr, int tl_per_block = 0, uint32_t* __restrict__ amax_part = nullptr) {
    constexpr bool GROUPED = !std::is_void<OutT1>::value;
    static_assert(!NARROW || (!GROUPED && !SPLIT), "narrow tiles: one problem, unsplit");
    using FoldT = typename std::conditional<GROUPED, OutT1, OutT>::type;
    static_assert(!AMAX_OUT || (!NARROW && (GROUPED || !SPLIT) &&
                                (std::is_same<FoldT, uint16_t>::value || std::is_same<FoldT, f16_t>::value ||
                                 std::is_same<FoldT, float>::value)),
                  "output absmax: 256x256 tiles, the unsplit single problem or a grouped launch's second "
                  "problem, bf16, f16 or fp32 output");
    using Out1 = typename std::conditional<GROUPED, OutT1, OutT>::type;
    constexpr int FM = NARROW ? 2 : 4, FN = 2;    // 32x32 MFMA tiles per wave
    constexpr int BN = NARROW ? 128 : kPBN;       // tile columns
    constexpr int WR = 32 * FM;                   // rows of a wave's part
    constexpr int NDA = 4, NDB = NARROW ? 2 : 4;  // A and B DMA instructions per wave and step
    using G0 = EpiGeom<(int)sizeof(OutT), FM>;
    using G1 = EpiGeom<(int)sizeof(Out1), FM>;
    constexpr int SLAB = G0::SLAB > G1::SLAB ? G0::SLAB : G1::SLAB;
    // after an epilogue, a wait that leaves the smaller store count in flight
    // (only where the wave's whole part -- 128x64, or 64x64 in narrow tiles
    // -- was in range: every store of an edge part sits behind a branch on
    // its lanes' range, so such a wave may have issued fewer, down to none,
    // and then waits for vmcnt(0))
    constexpr int NSTMIN = G0::NST < G1::NST ? G0::NST : G1::NST;
    constexpr int W_AFTER = NSTMIN > 63 ? 63 : NSTMIN;
    constexpr uint32_t kOOB = 0x80000000u;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * kPStage + kPBiasSlots * kPBiasSlot + 8 * SLAB];
    uint8_t* const lbias = lds + 2 * kPStage;

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = NARROW ? w >> 1 : w >> 2, wn = NARROW ? w & 1 : w & 3;
    // a stamp of the real-time counter (TIMELINE only; a vector store)
    auto stamp = [&](int idx) {
        if constexpr (TIMELINE) {
            if (w == 0 && idx < tl_per_block) {
                const uint64_t t = __builtin_amdgcn_s_memrealtime();
                if (lane == 0) tl[(int64_t)blockIdx.x * tl_per_block + idx] = t;
            }
        }
    };
    stamp(0);
    uint8_t* const slab = lds + 2 * kPStage + kPBiasSlots * kPBiasSlot + w * SLAB;
    // a 2-byte bias of odd length: its last element, which the dword bias DMA
    // cannot deliver (it shares a dword with the end of the buffer), read
    // once here rather than in every epilogue
    uint32_t bias_tail = 0;
    if (HAS_BIAS && sizeof(BiasT) == 2 && (N & 1))
        bias_tail = __builtin_amdgcn_readfirstlane(reinterpret_cast<const uint16_t*>(bias)[N - 1]);
    const int tiles_m = (M + kPBM - 1) / kPBM, tiles_n = (N + BN - 1) / BN;
    const int ntiles = tiles_m * tiles_n;
    const int nk = (K + kPKB - 1) / kPKB;
    const int P = gridDim.x;
    const int q = P >> 3, rr = P & 7;
    const int xcd = blockIdx.x & 7, idx = blockIdx.x >> 3;
    const int bl = xcd < rr ? xcd * (q + 1) + idx : rr * (q + 1) + (xcd - rr) * q + idx;
    // Work units: unit u of the nunits is (K slice u / ntiles, tile u % ntiles
    // of the grouped order); block bl takes units bl, bl+P, ...  Unsplit: one
    // slice of all nk steps.  SPLIT: nsplit slices of L = ksteps steps (the
    // last one shorter); a unit's fp32 partial tile goes to slice ks of C
    // ([nsplit][M][N], ldc = N).  Units running at the same time share a K
    // slice, so tiles of one row (column) meet their A (B) panel in L2.
    //
    // GROUPED: the units of a second GEMM p1 (unsplit tiles) follow in the
    // same grid, dealt by the static schedule of gemm_sched.hpp: this
    // problem's units round-robin first, then p1's in start-time order.
    const int L = SPLIT ? ksteps : nk;
    const int nunits = SPLIT ? ntiles * nsplit : ntiles;
    const int tiles_m1 = GROUPED ? (p1.M + kPBM - 1) / kPBM : 1, tiles_n1 = GROUPED ? (p1.N + kPBN - 1) / kPBN : 1;
    const int nk1 = GROUPED ? (p1.K + kPKB - 1) / kPKB : 0;
    const GroupSched gs{P, nunits, L + kUnitOverhead, GROUPED ? tiles_m1 * tiles_n1 : 0, nk1 + kUnitOverhead};
    const int my_tiles = GROUPED ? gs_d0(gs, bl) + gs_d1(gs, bl)
                                 : (bl < nunits ? (nunits - bl + P - 1) / P : 0);  // work units of this block
    auto tile_mn = [&](int r, int& pr, int& m0, int& n0, int& kb, int& nku, int& slot) {
        int lt = bl + r * P;
        pr = 0;
        if (GROUPED) gs_unit(gs, bl, r, pr, lt);
        slot = 0;
        if (SPLIT && pr == 0) {
            slot = lt / ntiles;
            lt -= slot * ntiles;
        }
        kb = slot * L;
        nku = pr ? nk1 : min(nk - kb, L);
        const int tm_ = pr ? tiles_m1 : tiles_m, tn_ = pr ? tiles_n1 : tiles_n;
        const int per_group = kGroupM * tn_;
        const int group = lt / per_group;
        const int first_m = group * kGroupM;
        const int gsize = min(tm_ - first_m, kGroupM);
        const int in_group = lt - group * per_group;
        m0 = (first_m + in_group % gsize) * kPBM;
        n0 = (in_group / gsize) * BN;
    };
    int S = 0;  // DMA steps of this block
    for (int r = 0; r < my_tiles; ++r) {
        int pr, m0, n0, kb, nku, slot;
        tile_mn(r, pr, m0, n0, kb, nku, slot);
        S += nku;
    }

    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, M * lda, 0x00020000);
    const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, N * ldb, 0x00020000);
    const __amdgpu_buffer_rsrc_t rA1 =
        __builtin_amdgcn_make_buffer_rsrc((void*)p1.A, (short)0, GROUPED ? p1.M * p1.lda : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t rB1 =
        __builtin_amdgcn_make_buffer_rsrc((void*)p1.B, (short)0, GROUPED ? p1.N * p1.ldb : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t rBias =
        __builtin_amdgcn_make_buffer_rsrc((void*)bias, (short)0, HAS_BIAS ? N * (int)sizeof(BiasT) : 0, 0x00020000);

    // ---- DMA.  Instruction d (0..3) of wave w fills rows (w*4+d)*8 + lane/8
    // of the stage's A and B parts; the lane's slot lane&7 takes global chunk
    // (lane&7) ^ swz(row), and swz(row) = 4*(d&1) + (lane>>4).  Each lane
    // keeps the byte offsets of its even- and odd-instruction rows; the
    // whole offset is the buffer's per-lane offset, so rows past M (N) are
    // outside the buffer's range and read as zero, and a chunk past K (or a
    // step past the block's last) gets an offset beyond any range.
    const int drow = lane >> 3;
    const int dch0 = ((lane & 7) ^ (lane >> 4)) << 4;
    const int dch1 = dch0 ^ 64;
    int d_tile = 0, d_k = 0, d_m0 = 0, d_n0 = 0, d_g = 0, d_kb = 0, d_nku = 0, d_slot = 0, d_p = 0;
    uint32_t oa0 = kOOB, oa1 = kOOB, ob0 = kOOB, ob1 = kOOB, obias = kOOB;
    auto dprep = [&]() {
        const bool live = d_g < S;
        const bool q1 = GROUPED && d_p;
        const int lda_ = q1 ? p1.lda : lda, ldb_ = q1 ? p1.ldb : ldb, K_ = q1 ? p1.K : K;
        const int kstep = d_kb + d_k;
        const int k0 = kstep * kPKB + dch0, k1 = kstep * kPKB + dch1;
        const uint32_t ra = (uint32_t)(d_m0 + w * 32 + drow), rb = (uint32_t)(d_n0 + w * 8 * NDB + drow);
        oa0 = (live && k0 < K_) ? ra * (uint32_t)lda_ + (uint32_t)k0 : kOOB;
        oa1 = (live && k1 < K_) ? (ra + 8u) * (uint32_t)lda_ + (uint32_t)k1 : kOOB;
        ob0 = (live && k0 < K_) ? rb * (uint32_t)ldb_ + (uint32_t)k0 : kOOB;
        ob1 = (live && k1 < K_) ? (rb + 8u) * (uint32_t)ldb_ + (uint32_t)k1 : kOOB;
        if (HAS_BIAS) obias = live ? (uint32_t)(d_n0 * (int)sizeof(BiasT) + w * 256 + lane * 4) : kOOB;
    };
    auto dissue = [&]() {
        uint8_t* base = lds + ((uint32_t)d_g & 1u) * kPStage;
        const bool q1 = GROUPED && d_p;
        const __amdgpu_buffer_rsrc_t ra_ = q1 ? rA1 : rA, rb_ = q1 ? rB1 : rB;
        const uint32_t a16 = 16u * (uint32_t)(q1 ? p1.lda : lda), b16 = 16u * (uint32_t)(q1 ? p1.ldb : ldb);
#pragma unroll
        for (int d = 0; d < 4; ++d)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra_, (__attribute__((address_space(3))) void*)(base + (w * 4 + d) * 1024), 16,
                ((d & 1) ? oa1 : oa0) + (uint32_t)(d >> 1) * a16, 0, 0, 0);
#pragma unroll
        for (int d = 0; d < NDB; ++d)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb_, (__attribute__((address_space(3))) void*)(base + kPBM * kPKB + (w * NDB + d) * 1024), 16,
                ((d & 1) ? ob1 : ob0) + (uint32_t)(d >> 1) * b16, 0, 0, 0);
        if (HAS_BIAS)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rBias,
                (__attribute__((address_space(3))) void*)(lbias + ((uint32_t)d_tile % kPBiasSlots) * kPBiasSlot +
                                                          w * 256),
                4, obias, 0, 0, 0);
    };
    // instruction k (0..NDA+NDB) of dissue(): A rows (4), B rows (NDB), bias
    auto dissue_one = [&](int k) __attribute__((always_inline)) {
        uint8_t* base = lds + ((uint32_t)d_g & 1u) * kPStage;
        const bool q1 = GROUPED && d_p;
        if (k < NDA) {
            const uint32_t a16 = 16u * (uint32_t)(q1 ? p1.lda : lda);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                q1 ? rA1 : rA, (__attribute__((address_space(3))) void*)(base + (w * 4 + k) * 1024), 16,
                ((k & 1) ? oa1 : oa0) + (uint32_t)(k >> 1) * a16, 0, 0, 0);
        } else if (k < NDA + NDB) {
            const int d = k - NDA;
            const uint32_t b16 = 16u * (uint32_t)(q1 ? p1.ldb : ldb);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                q1 ? rB1 : rB,
                (__attribute__((address_space(3))) void*)(base + kPBM * kPKB + (w * NDB + d) * 1024), 16,
                ((d & 1) ? ob1 : ob0) + (uint32_t)(d >> 1) * b16, 0, 0, 0);
        } else if (HAS_BIAS && d_k == 0) {  // a tile's bias, once, with its first step
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rBias,
                (__attribute__((address_space(3))) void*)(lbias + ((uint32_t)d_tile % kPBiasSlots) * kPBiasSlot +
                                                          w * 256),
                4, obias, 0, 0, 0);
        }
    };
    auto dadvance = [&]() {
        if (d_g < S && ++d_k == d_nku) {
            d_k = 0;
            if (++d_tile < my_tiles) tile_mn(d_tile, d_p, d_m0, d_n0, d_kb, d_nku, d_slot);
        }
        ++d_g;
        dprep();
    };
    if (my_tiles > 0) tile_mn(0, d_p, d_m0, d_n0, d_kb, d_nku, d_slot);
    dprep();

    // ---- fragments (v_mfma_f32_32x32x64_f8f6f4 operand layout: lane l
    // supplies row l%32, K bytes 32*(l/32) .. +32 of the 64-byte depth):
    // chunks 4e + 2*(l/32) and +1 of K-half e, from slots chunk ^ swz(row)
    const int fr = lane & 31;
    const int fsw = (fr >> 1) & 7;
    const int c0 = (lane >> 5) * 2;
    int foff[2][2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        foff[e][0] = fr * kPKB + (((4 * e + c0) ^ fsw) << 4);
        foff[e][1] = fr * kPKB + (((4 * e + c0 + 1) ^ fsw) << 4);
    }
    auto rd = [&](const uint8_t* p, int e) -> v8i {
        const u32x4 lo = *reinterpret_cast<const u32x4*>(p + foff[e][0]);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(p + foff[e][1]);
        v8i r;
        r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
        r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
        return r;
    };

    v16f acc[FM][FN];
    v8i fa0[FM], fb0[FN], fa1[FM], fb1[FN];
    int after_epi = 0, c_h = 0;
    uint32_t am_acc = 0;  // AMAX_OUT: this lane's biased fold of every value it stores
    const float sab = SPLIT ? 1.0f : sa[0] * sb[0];
    const float sab1 = GROUPED ? p1.sa[0] * p1.sb[0] : 0.0f;

    // One half-step: MFMAs on (fa, fb); fragments of half-step c_h+1 into
    // (na, nb).  Odd half-steps first wait for the DMA step that half-step
    // c_h+1 reads (after an epilogue its stores are still counted), then
    // synchronise the block and issue the DMA two steps ahead.
    //
    // Issue order, frozen by scheduling barriers: MFMA x (row block x/2,
    // column block x%2), then, for x < 4, three of the twelve fragment
    // reads, then (odd half-steps) this MFMA's share of the nine DMA
    // instructions -- two after MFMA 0, one after each later one (narrow
    // tiles: four MFMAs, two of the eight reads and two, two, two and one
    // of the seven DMA instructions under each).  The reads
    // all sit under the first four MFMAs, so they have landed by the end of
    // the half-step and the wait before the next barrier costs nothing; the
    // DMA is spread over the whole half-step instead of leaving as one burst
    // (with the compiler's own order, driven by scheduling hints only, the
    // reads and the DMA bunched up: the grouped backward ran 6% slower).
    auto half = [&](auto zero, auto odd, v8i* fa, v8i* fb, v8i* na, v8i* nb) {
        __builtin_amdgcn_sched_barrier(0);
        if (decltype(odd)::value) {
            if (after_epi == 1)
                __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(W_AFTER));
            else
                __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
            after_epi = 0;
            __builtin_amdgcn_s_barrier();
        }
        const int nxt = c_h + 1;
        const uint8_t* sA = lds + (((uint32_t)nxt >> 1) & 1u) * kPStage;
        const uint8_t* sB = sA + kPBM * kPKB;
        const int e = nxt & 1;
        constexpr int NR = 2 * (FM + FN);  // 16-byte fragment reads per half-step
        u32x4 part[NR];  // read r: fragment r/2 (A0..A(FM-1), B0, B1), 16-byte half r%2
#pragma unroll
        for (int x = 0; x < FM * FN; ++x) {
            const int i = x >> 1, j = x & 1;
            if (decltype(zero)::value) {
                const v16f z = {};
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[j], fa[i], z, FB, FA, 0, 0, 0, 0);
            } else {
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[j], fa[i], acc[i][j], FB, FA, 0, 0,
                                                                            0, 0);
            }
            if (x < 4) {
#pragma unroll
                for (int r = (NR / 4) * x; r < (NR / 4) * (x + 1); ++r) {
                    const int f = r >> 1, h = r & 1;
                    const uint8_t* p =
                        f < FM ? sA + (wm * WR + f * 32) * kPKB : sB + (wn * 64 + (f - FM) * 32) * kPKB;
                    part[r] = *reinterpret_cast<const u32x4*>(p + foff[e][h]);
                }
            }
            if (decltype(odd)::value) {
                if (NARROW) {  // seven instructions over four MFMAs: 2, 2, 2, 1
                    dissue_one(2 * x);
                    if (2 * x + 1 <= NDA + NDB) dissue_one(2 * x + 1);
                } else if (x == 0) {
                    dissue_one(0);
                    dissue_one(1);
                } else {
                    dissue_one(x + 1);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int f = 0; f < FM + FN; ++f) {
            const u32x4 lo = part[2 * f], hi = part[2 * f + 1];
            v8i r;
            r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
            r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
            if (f < FM) na[f] = r; else nb[f - FM] = r;
        }
        ++c_h;
        if (decltype(odd)::value) dadvance();
    };

    // Stores one finished tile: scale, bias, conversion to T, the slab pass
    // and the 16-byte row-segment stores (tile: this block's unit index, for
    // the bias slot).  Returns whether the wave's part lay wholly inside the
    // output, i.e. whether it issued all its stores.
    // always inlined: when both problems store the same type this lambda is
    // called from two places, and an outlined copy would take acc by
    // reference, i.e. through scratch memory
    auto store_tile = [&](auto tag, auto with_bias, auto fold, typename decltype(tag)::type* const Cu, int Mo,
                          int No, int ldco, int veco, float sabo, int tile, int tm0,
                          int tn0) __attribute__((always_inline)) {
        using T = typename decltype(tag)::type;
        constexpr bool BIAS = decltype(with_bias)::value;
        constexpr bool FOLD = AMAX_OUT && decltype(fold)::value;  // this problem's |C| goes into am_acc
        constexpr int ES = (int)sizeof(T);
        constexpr int SR = EpiGeom<ES>::SR, SROW = EpiGeom<ES>::SROW;
        constexpr int NPASS = EpiGeom<ES>::NPASS, SPP = EpiGeom<ES>::SPP;
        const int el = fresh_lane(), efr = el & 31;
        const int rowb = tm0 + wm * WR;
        const int colw = tn0 + wn * 64;
        const int h4 = (el >> 5) * 4;
        const uint8_t* bsl = lbias + ((uint32_t)tile % kPBiasSlots) * kPBiasSlot;
        // bias of the lane's columns colw + 32j + 8g + h4 + (0..3): fp32 as
        // values (bv), bf16 or f16 as the raw pairs (braw: 16 registers instead of
        // 32, widened where they are added, which keeps the forward's
        // epilogue within the register budget next to the next tile's
        // fragments).  A 2-byte bias of odd length: its last element shares a
        // dword with the end of the buffer, which the dword DMA returned as
        // zero, so it is patched in from bias_tail.
        constexpr bool PACKB = BIAS && sizeof(BiasT) == 2;
        float bv[FN][4][4];
        uint32_t braw[FN][4][2];
        const uint32_t tbits = bias_tail;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int lc = wn * 64 + j * 32 + 8 * g + h4;
                const int col = tn0 + lc;
                float b0 = 0.f, b1 = 0.f, b2 = 0.f, b3 = 0.f;
                uint32_t x0 = 0, x1 = 0;
                if (PACKB) {
                    const u32x2 v = *reinterpret_cast<const u32x2*>(bsl + lc * 2);
                    x0 = v.x;
                    x1 = v.y;
                    if (No & 1) {
                        x0 = col == No - 1 ? (x0 & 0xFFFF0000u) | tbits : x0;
                        x0 = col + 1 == No - 1 ? (x0 & 0xFFFFu) | (tbits << 16) : x0;
                        x1 = col + 2 == No - 1 ? (x1 & 0xFFFF0000u) | tbits : x1;
                        x1 = col + 3 == No - 1 ? (x1 & 0xFFFFu) | (tbits << 16) : x1;
                    }
                } else if (BIAS) {
                    const f32x4 v = *reinterpret_cast<const f32x4*>(bsl + lc * 4);
                    b0 = v.x; b1 = v.y; b2 = v.z; b3 = v.w;
                }
                bv[j][g][0] = b0; bv[j][g][1] = b1; bv[j][g][2] = b2; bv[j][g][3] = b3;
                braw[j][g][0] = x0; braw[j][g][1] = x1;
            }
        // slab read-back geometry: lane -> (row, 16-byte chunk)
        constexpr int CPR = 64 * ES / 16;
        constexpr int RPS = 64 / CPR;
        const int srow = el / CPR, rc = el % CPR;
        const int scol = colw + rc * (16 / ES);
        const bool col_full = veco && scol + 16 / ES <= No;
        const int my_sr = efr % SR, my_pass = efr / SR;
        typedef typename std::conditional<ES == 2, u32x2, f32x4>::type Pk;
        // LDS operations of one wave execute in order, so a pass's reads see
        // its writes and precede the next pass's writes; the empty asm
        // statements keep the compiler from reordering them.
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            Pk pk[FN][4];
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const v16f& a = acc[i][j];
                    float c0 = bv[j][g][0], c1 = bv[j][g][1], c2 = bv[j][g][2], c3 = bv[j][g][3];
                    if (PACKB && std::is_same<BiasT, f16_t>::value) {
                        // plain widening: a NaN bias makes a NaN output,
                        // whose payload the output conversion replaces
                        c0 = (float)__builtin_bit_cast(_Float16, (uint16_t)(braw[j][g][0] & 0xFFFFu));
                        c1 = (float)__builtin_bit_cast(_Float16, (uint16_t)(braw[j][g][0] >> 16));
                        c2 = (float)__builtin_bit_cast(_Float16, (uint16_t)(braw[j][g][1] & 0xFFFFu));
                        c3 = (float)__builtin_bit_cast(_Float16, (uint16_t)(braw[j][g][1] >> 16));
                    } else if (PACKB) {
                        c0 = __uint_as_float(braw[j][g][0] << 16);
                        c1 = __uint_as_float(braw[j][g][0] & 0xFFFF0000u);
                        c2 = __uint_as_float(braw[j][g][1] << 16);
                        c3 = __uint_as_float(braw[j][g][1] & 0xFFFF0000u);
                    }
                    const float v0 = a[4 * g] * sabo + c0, v1 = a[4 * g + 1] * sabo + c1;
                    const float v2 = a[4 * g + 2] * sabo + c2, v3 = a[4 * g + 3] * sabo + c3;
                    if constexpr (std::is_same<T, f16_t>::value)
                        pk[j][g] = u32x2{f32_to_f16_rne(v0) | (f32_to_f16_rne(v1) << 16),
                                         f32_to_f16_rne(v2) | (f32_to_f16_rne(v3) << 16)};
                    else if constexpr (ES == 2)
                        pk[j][g] = u32x2{pack_bf16_rne(v0, v1), pack_bf16_rne(v2, v3)};
                    else
                        pk[j][g] = f32x4{v0, v1, v2, v3};
                }
#pragma unroll
            for (int p = 0; p < NPASS; ++p) {
                if (my_pass == p) {
#pragma unroll
                    for (int j = 0; j < FN; ++j)
#pragma unroll
                        for (int g = 0; g < 4; ++g)
                            *reinterpret_cast<Pk*>(slab + my_sr * SROW + (j * 32 + 8 * g + h4) * ES) = pk[j][g];
                }
                asm volatile("" ::: "memory");
#pragma unroll
                for (int s = 0; s < SPP; ++s) {
                    const int sr = s * RPS + srow;
                    const u32x4 val = *reinterpret_cast<const u32x4*>(slab + sr * SROW + rc * 16);
                    const int row = rowb + i * 32 + p * SR + sr;
                    if (row < Mo) {
                        T* dst = Cu + (int64_t)row * ldco + scol;
                        if (col_full) {
                            if (veco == 2)
                                __builtin_nontemporal_store(val, reinterpret_cast<u32x4*>(dst));
                            else
                                *reinterpret_cast<u32x4*>(dst) = val;
                            if constexpr (FOLD && std::is_same<T, f16_t>::value) {
                                am_acc = fold_f16x2_biased(am_acc, val.x);
                                am_acc = fold_f16x2_biased(am_acc, val.y);
                                am_acc = fold_f16x2_biased(am_acc, val.z);
                                am_acc = fold_f16x2_biased(am_acc, val.w);
                            } else if constexpr (FOLD && ES == 2) {
                                am_acc = fold_bf16x2_biased(am_acc, val.x);
                                am_acc = fold_bf16x2_biased(am_acc, val.y);
                                am_acc = fold_bf16x2_biased(am_acc, val.z);
                                am_acc = fold_bf16x2_biased(am_acc, val.w);
                            } else if constexpr (FOLD) {
                                am_acc = fold_f32_biased(am_acc, val.x); am_acc = fold_f32_biased(am_acc, val.y);
                                am_acc = fold_f32_biased(am_acc, val.z); am_acc = fold_f32_biased(am_acc, val.w);
                            }
                        } else {
                            const T* ev = reinterpret_cast<const T*>(&val);
#pragma unroll
                            for (int x = 0; x < 16 / ES; ++x)
                                if (scol + x < No) {
                                    dst[x] = ev[x];
                                    if constexpr (FOLD && std::is_same<T, f16_t>::value)  // low half
                                        am_acc = fold_f16x2_biased(
                                            am_acc, (uint32_t)reinterpret_cast<const uint16_t*>(ev)[x]);
                                    else if constexpr (FOLD && ES == 2)  // the value in the low half
                                        am_acc = fold_bf16x2_biased(
                                            am_acc, (uint32_t)reinterpret_cast<const uint16_t*>(ev)[x]);
                                    else if constexpr (FOLD)
                                        am_acc = fold_f32_biased(am_acc, reinterpret_cast<const uint32_t*>(ev)[x]);
                                }
                        }
                    }
                }
                asm volatile("" ::: "memory");
            }
        }
        return rowb + 32 * FM <= Mo && colw + 64 <= No;
    };

    auto epilogue = [&](int tile) {
        int tp, tm0, tn0, tkb, tnku, tslot;
        tile_mn(tile, tp, tm0, tn0, tkb, tnku, tslot);
        bool whole;
        if (GROUPED && tp)
            whole = store_tile(Tag<Out1>{}, std::false_type{}, std::true_type{}, static_cast<Out1*>(p1.C), p1.M,
                               p1.N, p1.ldc, p1.vec_out, sab1, tile, tm0, tn0);
        else
            whole = store_tile(Tag<OutT>{}, std::integral_constant<bool, HAS_BIAS>{},
                               std::integral_constant<bool, !GROUPED>{},
                               SPLIT ? C + (int64_t)tslot * M * N : C, M, N, ldc, vec_out, sab, tile, tm0, tn0);
        after_epi = whole ? 1 : 2;
    };

    // prologue: DMA steps 0 and 1, fragments of half-step 0
    for (int g = 0; g < 2; ++g) {
        dissue();
        dadvance();
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(NDA + NDB + (HAS_BIAS ? 1 : 0)));
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int i = 0; i < FM; ++i) fa0[i] = rd(lds + (wm * WR + i * 32) * kPKB, 0);
#pragma unroll
    for (int j = 0; j < FN; ++j) fb0[j] = rd(lds + kPBM * kPKB + (wn * 64 + j * 32) * kPKB, 0);

    using Z = std::true_type;
    using NZ = std::false_type;
    using ODD = std::true_type;
    using EVEN = std::false_type;
    // a tile is 2*max(nk,1) half-steps; the fragments of its first half-step
    // are in (fa0, fb0) when it starts
    for (int tile = 0; tile < my_tiles; ++tile) {
        int up, um0, un0, ukb, unku, uslot;
        tile_mn(tile, up, um0, un0, ukb, unku, uslot);
        stamp(1 + 3 * tile);
        half(Z{}, EVEN{}, fa0, fb0, fa1, fb1);
        half(NZ{}, ODD{}, fa1, fb1, fa0, fb0);
        for (int k = 1; k < unku; ++k) {
            half(NZ{}, EVEN{}, fa0, fb0, fa1, fb1);
            half(NZ{}, ODD{}, fa1, fb1, fa0, fb0);
        }
        stamp(2 + 3 * tile);
        epilogue(tile);
        stamp(3 + 3 * tile);
    }
    if constexpr (AMAX_OUT) {  // every block, tiles or none, writes its 8 partials
        uint32_t m;
        if constexpr (std::is_same<FoldT, f16_t>::value) m = unbias_f16x2(am_acc);
        else if constexpr (sizeof(FoldT) == 2) m = unbias_bf16x2(am_acc);
        else m = unbias_f32(am_acc);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off, 64));
        if (lane == 0) amax_part[bl * 8 + w] = m;
    }
    __builtin_amdgcn_s_waitcnt(0);  // every DMA has landed before the block's LDS is released
}

template <int FA, int FB, typename OutT, typename BiasT, bool HAS_BIAS, bool SPLIT = false, typename OutT1 = void>
__global__ __launch_bounds__(512, 1) void gemm_nt_persistent_kernel(
    const uint8_t* __restrict__ A, int lda, const uint8_t* __restrict__ B, int ldb, int M, int N, int K,
    const float* __restrict__ sa, const float* __restrict__ sb, const BiasT* __restrict__ bias,
    OutT* __restrict__ C, int ldc, int vec_out, int ksteps = 0, int nsplit = 1, PProb p1 = {}) {
    persistent_body<FA, FB, OutT, BiasT, HAS_BIAS, SPLIT, OutT1, false>(A, lda, B, ldb, M, N, K, sa, sb, bias, C,
                                                                        ldc, vec_out, ksteps, nsplit, p1);
}

// The forward kernel with the per-tile timeline (df_fp8_gemm_fwd_timeline).
template <int FA, int FB, typename OutT, typename BiasT, bool HAS_BIAS>
__global__ __launch_bounds__(512, 1) void gemm_nt_persistent_timeline_kernel(
    const uint8_t* __restrict__ A, int lda, const uint8_t* __restrict__ B, int ldb, int M, int N, int K,
    const float* __restrict__ sa, const float* __restrict__ sb, const BiasT* __restrict__ bias,
    OutT* __restrict__ C, int ldc, int vec_out, uint64_t* __restrict__ tl, int tl_per_block) {
    persistent_body<FA, FB, OutT, BiasT, HAS_BIAS, false, void, false, true>(
        A, lda, B, ldb, M, N, K, sa, sb, bias, C, ldc, vec_out, 0, 1, PProb{}, tl, tl_per_block);
}

template <int FA, int FB, typename OutT, typename BiasT, bool HAS_BIAS>
__global__ __launch_bounds__(512, 1) void gemm_nt_persistent_amax_kernel(
    const uint8_t* __restrict__ A, int lda, const uint8_t* __restrict__ B, int ldb, int M, int N, int K,
    const float* __restrict__ sa, const float* __restrict__ sb, const BiasT* __restrict__ bias,
    OutT* __restrict__ C, int ldc, int vec_out, uint32_t* __restrict__ amax_part) {
    persistent_body<FA, FB, OutT, BiasT, HAS_BIAS, false, void, false, false, true>(
        A, lda, B, ldb, M, N, K, sa, sb, bias, C, ldc, vec_out, 0, 1, PProb{}, nullptr, 0, amax_part);
}

// The grouped dX + dW launch that also folds |dX| (df_fp8_gemm_bwd_absmax).
template <int FA, int FB, typename OutT, bool SPLIT, typename OutT1>
__global__ __launch_bounds__(512, 1) void gemm_nt_persistent_grouped_amax_kernel(
    const uint8_t* __restrict__ A, int lda, const uint8_t* __restrict__ B, int ldb, int M, int N, int K,
    const float* __restrict__ sa, const float* __restrict__ sb, OutT* __restrict__ C, int ldc, int vec_out,
    int ksteps, int nsplit, PProb p1, uint32_t* __restrict__ amax_part) {
    persistent_body<FA, FB, OutT, float, false, SPLIT, OutT1, false, false, true>(
        A, lda, B, ldb, M, N, K, sa, sb, nullptr, C, ldc, vec_out, ksteps, nsplit, p1, nullptr, 0, amax_part);
}

template <int FA, int FB, typename OutT, typename BiasT, bool HAS_BIAS>
__global__ __launch_bounds__(512, 1) void gemm_nt_persistent_narrow_kernel(
    const uint8_t* __restrict__ A, int lda, const uint8_t* __restrict__ B, int ldb, int M, int N, int K,
    const float* __restrict__ sa, const float* __restrict__ sb, const BiasT* __restrict__ bias,
    OutT* __restrict__ C, int ldc, int vec_out) {
    persistent_body<FA, FB, OutT, BiasT, HAS_BIAS, false, void, true>(A, lda, B, ldb, M, N, K, sa, sb, bias, C, ldc,
                                                                      vec_out, 0, 1, PProb{});
}

// out[m,n] = (sum_s P[s][m][n]) * sa * sb + bias[n], slices in order; four
// consecutive columns per thread (16-byte partial loads) when N % 4 == 0.
template <typename OutT, typename BiasT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ P, int S, int M,
                                                            int N, const float* __restrict__ sa,
                                                            const float* __restrict__ sb,
                                                            const BiasT* __restrict__ bias,
                                                            OutT* __restrict__ C, int ldc, bool vec) {
    const float sab = sa[0] * sb[0];
    const int64_t total = (int64_t)M * N;
    const int64_t stride = (int64_t)gridDim.x * 256;
    if (vec) {
        for (int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4; e < total; e += stride * 4) {
            f32x4 acc = *reinterpret_cast<const f32x4*>(P + e);
            for (int s = 1; s < S; ++s) acc += *reinterpret_cast<const f32x4*>(P + (int64_t)s * total + e);
            const int m = (int)(e / N), n = (int)(e - (int64_t)m * N);
            float v[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = v[r] * sab + (bias ? bias_ld(bias, n + r) : 0.0f);
            store4(C + (int64_t)m * ldc + n, v);
        }
        return;
    }
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += stride) {
        float acc = P[e];
        for (int s = 1; s < S; ++s) acc += P[(int64_t)s * total + e];
        const int m = (int)(e / N), n = (int)(e - (int64_t)m * N);
        const float bv = bias ? bias_ld(bias, n) : 0.0f;
        C[(int64_t)m * ldc + n] = OutCvt<OutT>::cvt(acc * sab + bv);
    }
}

struct GemmArgs {
    const uint8_t* A; int lda;
    const uint8_t* B; int ldb;
    int M, N, K;
    const float* sa; const float* sb;
    const void* bias; void* C; int ldc;
    float* ws; size_t ws_bytes;
    hipStream_t st;
};

// Launch plan: tile configuration and split-K factor from a rounds cost
// model.  A 256x256 block (8 waves) occupies a CU alone: 256 tiles per
// round.  128x128 blocks (4 waves) run two per CU: 512 per round, each
// round doing half the work of a 256x256 round at about 85% of its
// per-CU rate (measured on the GPT-2 XL/small Linear shapes).  Cost is in
// units of one 256x256 K-step (128 bytes): rounds x (K-steps per slice +
// a fixed per-tile overhead), plus, for split-K, the partial-tile traffic
// ((S + 1) * M * N fp32 at roughly two K-steps per 10 MB).
struct GemmPlan {
    bool big;  // 256x256 (true) or 128x128
    int split;
};

static GemmPlan plan_gemm(int M, int N, int K, size_t ws_bytes) {
    constexpr double kOverheadSteps = 3.0;
    constexpr double kSmallRate = 0.59;  // (1/2) / 0.85
    const int nk = (K + kBK - 1) / kBK;
    const int64_t t256 = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
    const int64_t t128 = (int64_t)((M + 127) / 128) * ((N + 127) / 128);
    const double red_steps_per_byte = 2.0 / 10e6;
    GemmPlan best{true, 1};
    double best_cost = 1e300;
    for (int big = 1; big >= 0; --big) {
        if (big && (M < 256 || N < 256)) continue;
        const int64_t tiles = big ? t256 : t128;
        const int64_t slots = big ? 256 : 512;
        for (int s = 1; s <= 8; ++s) {
            if (s > 1 && (nk / s < 4 || (size_t)s * M * N * sizeof(float) > ws_bytes)) break;
            const double rounds = (double)((tiles * s + slots - 1) / slots);
            double cost = rounds * ((nk + s - 1) / s + kOverheadSteps) * (big ? 1.0 : kSmallRate);
            if (s > 1) cost += (double)(s + 1) * M * N * sizeof(float) * red_steps_per_byte;
            if (cost < best_cost * 0.97) {
                best_cost = cost;
                best = GemmPlan{big != 0, s};
            }
        }
    }
    return best;
}

static int plan_split(int M, int N, int K, size_t ws_bytes) { return plan_gemm(M, N, K, ws_bytes).split; }

template <int BM, int BN, int WM, int WN, int FA, int FB, typename OutT, typename BiasT>
static void launch_cfg(const GemmArgs& g) {
    const int tiles_m = (g.M + BM - 1) / BM, tiles_n = (g.N + BN - 1) / BN;
    const int tiles = tiles_m * tiles_n;
    const int nk = (g.K + kBK - 1) / kBK;
    const int S = plan_gemm(g.M, g.N, g.K, g.ws ? g.ws_bytes : 0).split;
    // vector epilogue stores need 4-element groups to stay aligned
    const bool vec_out = ((int64_t)g.ldc * (int64_t)sizeof(OutT)) % 16 == 0 && aligned16(g.C);
    // buffer-resource ranges are 32-bit byte counts
    const bool dma_ok = (int64_t)g.M * g.lda < (1ll << 31) && (int64_t)g.N * g.ldb < (1ll << 31);
    if (S == 1 && dma_ok) {
        gemm_nt_dma128_kernel<BM, BN, WM, WN, FA, FB, OutT, BiasT, false><<<tiles, 64 * WM * WN, 0, g.st>>>(
            g.A, g.lda, g.B, g.ldb, g.M, g.N, g.K, g.K, g.sa, g.sb, static_cast<const BiasT*>(g.bias),
            static_cast<OutT*>(g.C), g.ldc, vec_out, nullptr);
        return;
    }
    if (S == 1) {
        gemm_nt_kernel<BM, BN, WM, WN, FA, FB, OutT, BiasT, false><<<tiles, 64 * WM * WN, 0, g.st>>>(
            g.A, g.lda, g.B, g.ldb, g.M, g.N, g.K, g.K, g.sa, g.sb, static_cast<const BiasT*>(g.bias),
            static_cast<OutT*>(g.C), g.ldc, vec_out, nullptr);
        return;
    }
    const int kps = ((nk + S - 1) / S) * kBK;
    const int S_eff = (g.K + kps - 1) / kps;
    if (dma_ok)
        gemm_nt_dma128_kernel<BM, BN, WM, WN, FA, FB, OutT, BiasT, true><<<dim3(tiles, S_eff), 64 * WM * WN, 0, g.st>>>(
            g.A, g.lda, g.B, g.ldb, g.M, g.N, g.K, kps, g.sa, g.sb, static_cast<const BiasT*>(g.bias),
            static_cast<OutT*>(g.C), g.ldc, false, g.ws);
    else
        gemm_nt_kernel<BM, BN, WM, WN, FA, FB, OutT, BiasT, true><<<dim3(tiles, S_eff), 64 * WM * WN, 0, g.st>>>(
            g.A, g.lda, g.B, g.ldb, g.M, g.N, g.K, kps, g.sa, g.sb, static_cast<const BiasT*>(g.bias),
            static_cast<OutT*>(g.C), g.ldc, false, g.ws);
    const int64_t total = (int64_t)g.M * g.N;
    int blocks = (int)std::min<int64_t>((total + 255) / 256, 4096);
    const bool vec_red = (g.N % 4 == 0) && vec_out;
    splitk_reduce_kernel<OutT, BiasT><<<blocks, 256, 0, g.st>>>(g.ws, S_eff, g.M, g.N, g.sa, g.sb,
                                                                static_cast<const BiasT*>(g.bias),
                                                                static_cast<OutT*>(g.C), g.ldc, vec_red);
}

// Store mode of the persistent kernel's epilogue: 0 element stores, 1
// 16-byte stores, 2 16-byte non-temporal stores.  One store instruction
// writes whole 64-column row segments (128 bytes of bf16, 256 of fp32);
// non-temporal stores are kept to rows that start on a 128-byte boundary, so
// that no cache line is written in parts by several non-temporal stores (in
// a probe that did so -- 8-byte non-temporal stores -- one output of sixteen
// came back different, where plain stores matched).
static int epi_store_mode(const void* C, int64_t ldc_bytes) {
    if (ldc_bytes % 16 != 0 || !aligned16(C)) return 0;
    return (ldc_bytes % 128 == 0 && ((uintptr_t)C & 127u) == 0) ? 2 : 1;
}

// The persistent kernel takes outputs with at least one 256x256 tile per CU
// (smaller ones keep the split-K plan below).  Its per-lane buffer offsets
// reach a tile past the last row, so M*lda and N*ldb stay below 2^31 (and
// lda, ldb below 2^23); its bias DMA reads whole dwords.
static bool persistent_ok(const GemmArgs& g) {
    if ((int64_t)g.M * g.lda >= (1ll << 31) || (int64_t)g.N * g.ldb >= (1ll << 31)) return false;
    if (g.lda >= (1 << 23) || g.ldb >= (1 << 23)) return false;
    return !g.bias || aligned4(g.bias);
}

// Outputs with fewer 256x256 tiles than CUs (the dW GEMMs): the persistent
// kernel over S K slices of L DMA steps (S * tiles work units, fp32 partial
// tiles, then splitk_reduce_kernel sums the slices in order), S from the
// rounds cost model of plan_gemm in units of one 128-byte K step of a
// 256x256 tile plus the partial-tile traffic.  S = 1: one unit per tile.
// (A stream-K cut into equal per-CU ranges balanced the rounds better but
// ran 25% slower on the GPT-2 XL dW shapes: the CUs then read their A and B
// panels at unrelated K offsets and L2 reuse was lost.)
struct PSplit {
    int S, L;
    double cost;  // rounds cost model, in K steps of a 256x256 tile
};

static PSplit persistent_split_plan(int M, int N, int K, size_t ws_bytes, int cus) {
    constexpr double kOverheadSteps = 3.0;
    const double red_steps_per_byte = 2.0 / 10e6;
    const int nk = (K + kPKB - 1) / kPKB;
    const int64_t tiles = (int64_t)((M + kPBM - 1) / kPBM) * ((N + kPBN - 1) / kPBN);
    PSplit best{1, nk, (double)((tiles + cus - 1) / cus) * (nk + kOverheadSteps)};
    double best_cost = best.cost;
    for (int s = 2; s <= 8; ++s) {
        const int span = (nk + s - 1) / s;
        if (span < 4) break;
        const int se = (nk + span - 1) / span;
        if ((size_t)se * M * N * sizeof(float) > ws_bytes) break;
        const double rounds = (double)((tiles * se + cus - 1) / cus);
        const double cost =
            rounds * (span + kOverheadSteps) + (double)(se + 1) * M * N * sizeof(float) * red_steps_per_byte;
        if (cost < best_cost * 0.97) {
            best_cost = cost;
            best = PSplit{se, span, cost};
        }
    }
    return best;
}

template <int FA, int FB, typename OutT, typename BiasT>
static void launch_persistent(const GemmArgs& g, int grid) {
    const int vec_out = epi_store_mode(g.C, (int64_t)g.ldc * (int64_t)sizeof(OutT));
    if (g.bias)
        gemm_nt_persistent_kernel<FA, FB, OutT, BiasT, true><<<grid, 512, 0, g.st>>>(
            g.A, g.lda, g.B, g.ldb, g.M, g.N, g.K, g.sa, g.sb, static_cast<const BiasT*>(g.bias),
            static_cast<OutT*>(g.C), g.ldc, vec_out);
    else
        gemm_nt_persistent_kernel<FA, FB, OutT, BiasT, false><<<grid, 512, 0, g.st>>>(
            g.A, g.lda, g.B, g.ldb, g.M, g.N, g.K, g.sa, g.sb, nullptr, static_cast<OutT*>(g.C), g.ldc, vec_out);
}

template <int FA, int FB, typename OutT, typename BiasT>
static void launch_persistent_narrow(const GemmArgs& g, int grid) {
    const int vec_out = epi_store_mode(g.C, (int64_t)g.ldc * (int64_t)sizeof(OutT));
    if (g.bias)
        gemm_nt_persistent_narrow_kernel<FA, FB, OutT, BiasT, true><<<grid, 512, 0, g.st>>>(
            g.A, g.lda, g.B, g.ldb, g.M, g.N, g.K, g.sa, g.sb, static_cast<const BiasT*>(g.bias),
            static_cast<OutT*>(g.C), g.ldc, vec_out);
    else
        gemm_nt_persistent_narrow_kernel<FA, FB, OutT, BiasT, false><<<grid, 512, 0, g.st>>>(
            g.A, g.lda, g.B, g.ldb, g.M, g.N, g.K, g.sa, g.sb, nullptr, static_cast<OutT*>(g.C), g.ldc, vec_out);
}

// Narrow (256x128) tiles in the rounds cost model: a K step costs
// kNarrowStep of a 256x256 step, a tile kNarrowOverhead steps beyond them.
// Measured (bf16 output, 20 launches each): where both tilings run one
// round, narrow tiles took 0.75-0.77 of the time (GPT-2 small attn/mlp
// projections at 8192 tokens: about 0.74 per step and 2.5 per tile).  The
// smaller constants here also send the GPT-2 small c_attn and c_fc shapes,
// whose 256x256 plans end in a partly empty round, to narrow tiles (0-4%
// faster there), while the GPT-2 XL shapes at 16384 tokens keep 256x256
// tiles (narrow ones 13-40% slower).
constexpr double kNarrowStep = 0.6, kNarrowOverhead = 2.0;

// The kernel one NT GEMM call runs (df_fp8_gemm_nt_plan reports it): the
// persistent kernel when its offsets fit (split into K-slice units when the
// output has fewer tiles than CUs and a workspace allows it; its 256x128
// tiles when the rounds cost model puts them 3% below), otherwise the
// tiled kernels -- LDS-DMA when both operands fit a 32-bit buffer range,
// register-staged beyond -- with 256x256 or 128x128 blocks and split-K from
// plan_gemm.  Every launch below follows this plan.
struct NtPlan {
    int kind;   // DF_GEMM_KERNEL_*
    int split;  // K slices (1 = unsplit)
    int L;      // persistent split: DMA steps per slice
    int grid;   // persistent: blocks
};

static NtPlan nt_plan(const GemmArgs& g) {
    const int cus = device_cu_count();
    const size_t ws = g.ws ? g.ws_bytes : 0;
    if (cus > 0 && persistent_ok(g)) {
        const int tm = (g.M + kPBM - 1) / kPBM, nk = (g.K + kPKB - 1) / kPKB;
        const int64_t tiles = (int64_t)tm * ((g.N + kPBN - 1) / kPBN);
        const int64_t tiles_nw = (int64_t)tm * ((g.N + 127) / 128);
        NtPlan wide;
        double wcost;
        if (tiles >= cus) {
            wide = NtPlan{DF_GEMM_KERNEL_PERSISTENT, 1, 0, cus};
            wcost = (double)((tiles + cus - 1) / cus) * (nk + 3.0);
        } else {
            const PSplit ps = persistent_split_plan(g.M, g.N, g.K, ws, cus);
            wide = ps.S == 1 ? NtPlan{DF_GEMM_KERNEL_PERSISTENT, 1, 0, (int)tiles}
                             : NtPlan{DF_GEMM_KERNEL_PERSISTENT, ps.S, ps.L, (int)std::min<int64_t>(tiles * ps.S, cus)};
            wcost = ps.cost;
        }
        const double ncost = (double)((tiles_nw + cus - 1) / cus) * (nk * kNarrowStep + kNarrowOverhead);
        if (ncost < wcost * 0.97)
            return NtPlan{DF_GEMM_KERNEL_PERSISTENT_NARROW, 1, 0, (int)std::min<int64_t>(tiles_nw, cus)};
        return wide;
    }
    const GemmPlan gp = plan_gemm(g.M, g.N, g.K, ws);
    const bool dma_ok = (int64_t)g.M * g.lda < (1ll << 31) && (int64_t)g.N * g.ldb < (1ll << 31);
    const int kind = dma_ok ? (gp.big ? DF_GEMM_KERNEL_TILED_DMA_256 : DF_GEMM_KERNEL_TILED_DMA_128)
                            : (gp.big ? DF_GEMM_KERNEL_TILED_REG_256 : DF_GEMM_KERNEL_TILED_REG_128);
    int split = gp.split;
    if (split > 1) {  // the slice count the launch really makes
        const int nk = (g.K + kBK - 1) / kBK;
        const int kps = ((nk + split - 1) / split) * kBK;
        split = (g.K + kps - 1) / kps;
    }
    return NtPlan{kind, split, 0, 0};
}

template <int FA, int FB, typename OutT, typename BiasT>
static void launch_shape(const GemmArgs& g) {
    const NtPlan p = nt_plan(g);
    if (p.kind == DF_GEMM_KERNEL_PERSISTENT_NARROW) {
        launch_persistent_narrow<FA, FB, OutT, BiasT>(g, p.grid);
        return;
    }
    if (p.kind == DF_GEMM_KERNEL_PERSISTENT) {
        if (p.split == 1) {
            launch_persistent<FA, FB, OutT, BiasT>(g, p.grid);
            return;
        }
        gemm_nt_persistent_kernel<FA, FB, float, BiasT, false, true><<<p.grid, 512, 0, g.st>>>(
            g.A, g.lda, g.B, g.ldb, g.M, g.N, g.K, g.sa, g.sb, nullptr, g.ws, g.N,
            epi_store_mode(g.ws, (int64_t)g.N * 4), p.L, p.split);
        const int64_t total = (int64_t)g.M * g.N;
        const int blocks = (int)std::min<int64_t>((total + 255) / 256, 4096);
        const bool vec_red = (g.N % 4 == 0) && ((int64_t)g.ldc * (int64_t)sizeof(OutT)) % 16 == 0 && aligned16(g.C);
        splitk_reduce_kernel<OutT, BiasT><<<blocks, 256, 0, g.st>>>(g.ws, p.split, g.M, g.N, g.sa, g.sb,
                                                                    static_cast<const BiasT*>(g.bias),
                                                                    static_cast<OutT*>(g.C), g.ldc, vec_red);
        return;
    }
    if (p.kind == DF_GEMM_KERNEL_TILED_DMA_256 || p.kind == DF_GEMM_KERNEL_TILED_REG_256)
        launch_cfg<256, 256, 2, 4, FA, FB, OutT, BiasT>(g);
    else
        launch_cfg<128, 128, 2, 2, FA, FB, OutT, BiasT>(g);
}

// Grouped backward launch: dW (problem 0, in S K slices when that balances
// better) and dX (problem 1) in one persistent grid of `cus` blocks, dealt by
// the static schedule of gemm_sched.hpp.  The plan compares, in the rounds
// cost model's steps, the schedule's makespan (plus the slice reduce) with
// the two launches it replaces: dX's rounds plus dW's own plan.
struct GroupPlan {
    bool grouped;
    int S, L;
};

static int64_t group_makespan(int cus, int64_t units0, int c0, int64_t units1, int c1) {
    const GroupSched gs{cus, (int)units0, c0, (int)units1, c1};
    int64_t mk = 0;
    for (int b = 0; b < cus; ++b) mk = std::max(mk, gs_finish(gs, b));
    return mk;
}

static GroupPlan grouped_plan(const GemmArgs& dw, const GemmArgs& dx, size_t ws_bytes, int cus) {
    constexpr double kOverheadSteps = kUnitOverhead;
    const double red_steps_per_byte = 2.0 / 10e6;
    const int nk0 = (dw.K + kPKB - 1) / kPKB, nk1 = (dx.K + kPKB - 1) / kPKB;
    // Where df_fp8_gemm_bwd_dx, given this workspace, cuts dX's reduction into
    // K slices (a small dX with a long reduction), dX is left to that call:
    // the grouped launch never slices dX, and this keeps dX bit-identical
    // between the two entry points.
    GemmArgs dxs = dx;
    dxs.ws = ws_bytes ? reinterpret_cast<float*>(uintptr_t{16}) : nullptr;  // only its presence is read
    dxs.ws_bytes = ws_bytes;
    if (nt_plan(dxs).split > 1) return GroupPlan{false, 1, nk0};
    const int64_t t0 = (int64_t)((dw.M + kPBM - 1) / kPBM) * ((dw.N + kPBN - 1) / kPBN);
    const int64_t t1 = (int64_t)((dx.M + kPBM - 1) / kPBM) * ((dx.N + kPBN - 1) / kPBN);
    // the two launches it replaces
    double separate = (double)((t1 + cus - 1) / cus) * (nk1 + kOverheadSteps);
    if (t0 >= cus) {
        separate += (double)((t0 + cus - 1) / cus) * (nk0 + kOverheadSteps);
    } else {
        const PSplit ps = persistent_split_plan(dw.M, dw.N, dw.K, ws_bytes, cus);
        separate += (double)((t0 * ps.S + cus - 1) / cus) * (ps.L + kOverheadSteps);
        if (ps.S > 1) separate += (double)(ps.S + 1) * dw.M * dw.N * sizeof(float) * red_steps_per_byte;
    }
    GroupPlan best{false, 1, nk0};
    double best_cost = separate;
    for (int s = 1; s <= 8; ++s) {
        const int span = (nk0 + s - 1) / s;
        if (s > 1 && span < 4) break;
        const int se = (nk0 + span - 1) / span;
        if (se > 1 && (size_t)se * dw.M * dw.N * sizeof(float) > ws_bytes) break;
        double cost = (double)group_makespan(cus, t0 * se, span + kUnitOverhead, t1, nk1 + kUnitOverhead);
        if (se > 1) cost += (double)(se + 1) * dw.M * dw.N * sizeof(float) * red_steps_per_byte;
        if (cost < best_cost * 0.97) {
            best_cost = cost;
            best = GroupPlan{true, se, span};
        }
    }
    return best;
}

// amax_part non-NULL: the launch also folds |dX| into 8 partials per block
// (grid = cus), for df_fp8_gemm_bwd_absmax.
template <typename DwT, typename DxT>
static void launch_grouped(const GemmArgs& dw, const GemmArgs& dx, const GroupPlan& gp, int cus,
                           uint32_t* amax_part = nullptr) {
    const PProb p1{dx.A, dx.B, dx.C, dx.sa, dx.sb, dx.lda, dx.ldb, dx.M, dx.N, dx.K, dx.ldc,
                   epi_store_mode(dx.C, (int64_t)dx.ldc * (int64_t)sizeof(DxT))};
    constexpr bool FOLDS =
        std::is_same<DxT, uint16_t>::value || std::is_same<DxT, f16_t>::value || std::is_same<DxT, float>::value;
    if (gp.S == 1) {
        const int vec_out = epi_store_mode(dw.C, (int64_t)dw.ldc * (int64_t)sizeof(DwT));
        if constexpr (FOLDS) {
            if (amax_part) {
                gemm_nt_persistent_grouped_amax_kernel<E5M2, E4M3, DwT, false, DxT><<<cus, 512, 0, dw.st>>>(
                    dw.A, dw.lda, dw.B, dw.ldb, dw.M, dw.N, dw.K, dw.sa, dw.sb, static_cast<DwT*>(dw.C), dw.ldc,
                    vec_out, 0, 1, p1, amax_part);
                return;
            }
        }
        gemm_nt_persistent_kernel<E5M2, E4M3, DwT, float, false, false, DxT><<<cus, 512, 0, dw.st>>>(
            dw.A, dw.lda, dw.B, dw.ldb, dw.M, dw.N, dw.K, dw.sa, dw.sb, nullptr, static_cast<DwT*>(dw.C), dw.ldc,
            vec_out, 0, 1, p1);
        return;
    }
    bool launched = false;
    if constexpr (FOLDS) {
        if (amax_part) {
            gemm_nt_persistent_grouped_amax_kernel<E5M2, E4M3, float, true, DxT><<<cus, 512, 0, dw.st>>>(
                dw.A, dw.lda, dw.B, dw.ldb, dw.M, dw.N, dw.K, dw.sa, dw.sb, dw.ws, dw.N,
                epi_store_mode(dw.ws, (int64_t)dw.N * 4), gp.L, gp.S, p1, amax_part);
            launched = true;
        }
    }
    if (!launched)
        gemm_nt_persistent_kernel<E5M2, E4M3, float, float, false, true, DxT><<<cus, 512, 0, dw.st>>>(
            dw.A, dw.lda, dw.B, dw.ldb, dw.M, dw.N, dw.K, dw.sa, dw.sb, nullptr, dw.ws, dw.N,
            epi_store_mode(dw.ws, (int64_t)dw.N * 4), gp.L, gp.S, p1);
    const int64_t total = (int64_t)dw.M * dw.N;
    const int blocks = (int)std::min<int64_t>((total + 255) / 256, 4096);
    const bool vec_red = (dw.N % 4 == 0) && ((int64_t)dw.ldc * (int64_t)sizeof(DwT)) % 16 == 0 && aligned16(dw.C);
    splitk_reduce_kernel<DwT, float><<<blocks, 256, 0, dw.st>>>(dw.ws, gp.S, dw.M, dw.N, dw.sa, dw.sb, nullptr,
                                                                 static_cast<DwT*>(dw.C), dw.ldc, vec_red);
}

// output and bias element types (nt_args admits: fp32 or bf16 output with
// an fp32 or bf16 bias, f16 output with an fp32 or f16 bias)
template <int FA, int FB>
static void dispatch_out(const GemmArgs& g, int bias_dtype, int c_dtype) {
    const bool bf16_bias = g.bias && bias_dtype == DF_DTYPE_BFLOAT16;
    const bool f16_bias = g.bias && bias_dtype == DF_DTYPE_HALF;
    if (c_dtype == DF_DTYPE_FLOAT32) {
        if (bf16_bias) launch_shape<FA, FB, float, uint16_t>(g);
        else launch_shape<FA, FB, float, float>(g);
    } else if (c_dtype == DF_DTYPE_HALF) {
        if (f16_bias) launch_shape<FA, FB, f16_t, f16_t>(g);
        else launch_shape<FA, FB, f16_t, float>(g);
    } else {
        if (bf16_bias) launch_shape<FA, FB, uint16_t, uint16_t>(g);
        else launch_shape<FA, FB, uint16_t, float>(g);
    }
}

}  // namespace dfk

using namespace dfk;

extern "C" size_t df_fp8_gemm_workspace_bytes(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    const int Kp = (K + 15) & ~15;
    // the larger of the two plans' needs: the persistent split (when the
    // operands fit its offsets) and the tiled kernels' split
    const int S = plan_split(M, N, Kp, SIZE_MAX);
    size_t need = S > 1 ? (size_t)S * (size_t)M * (size_t)N * sizeof(float) : 0;
    const int cus = device_cu_count();
    if (cus > 0) {
        const int64_t tiles = (int64_t)((M + kPBM - 1) / kPBM) * ((N + kPBN - 1) / kPBN);
        if (tiles < cus) {
            const PSplit ps = persistent_split_plan(M, N, Kp, SIZE_MAX, cus);
            if (ps.S > 1) need = std::max(need, (size_t)ps.S * (size_t)M * (size_t)N * sizeof(float));
        }
    }
    return need;
}

// Argument checks of one NT GEMM; on success fills g (empty: nothing to
// compute, M or N is 0).
static int nt_args(const char* fn, int fmt_a, const uint8_t* A, int lda, int fmt_b, const uint8_t* B, int ldb,
                   int M, int N, int K, const float* scale_a_dev, const float* scale_b_dev, int bias_dtype,
                   const void* bias, int c_dtype, void* C, int ldc, void* ws, size_t ws_bytes, void* stream,
                   GemmArgs& g, bool& empty) {
    DF_CHECK(M >= 0 && N >= 0 && K >= 0, DF_ERR_INVALID, "%s: negative size M=%d N=%d K=%d", fn, M, N, K);
    DF_CHECK((fmt_a == E4M3 || fmt_a == E5M2) && (fmt_b == E4M3 || fmt_b == E5M2), DF_ERR_UNSUPPORTED,
             "%s: bad fp8 formats %d %d", fn, fmt_a, fmt_b);
    DF_CHECK(c_dtype == DF_DTYPE_FLOAT32 || c_dtype == DF_DTYPE_BFLOAT16 || c_dtype == DF_DTYPE_HALF,
             DF_ERR_UNSUPPORTED, "%s: output dtype %d not supported", fn, c_dtype);
    DF_CHECK(!bias || bias_dtype == DF_DTYPE_FLOAT32 || bias_dtype == DF_DTYPE_BFLOAT16 || bias_dtype == DF_DTYPE_HALF,
             DF_ERR_UNSUPPORTED, "%s: bias dtype %d not supported", fn, bias_dtype);
    DF_CHECK(!bias || (bias_dtype == DF_DTYPE_HALF) == (c_dtype == DF_DTYPE_HALF) || bias_dtype == DF_DTYPE_FLOAT32,
             DF_ERR_UNSUPPORTED, "%s: bias dtype %d with output dtype %d not supported", fn, bias_dtype, c_dtype);
    DF_CHECK(ldc >= N, DF_ERR_INVALID, "%s: ldc=%d < N=%d", fn, ldc, N);
    empty = M == 0 || N == 0;
    if (empty) return DF_OK;
    DF_CHECK(A && B && C && scale_a_dev && scale_b_dev, DF_ERR_INVALID, "%s: NULL pointer", fn);
    DF_CHECK(lda >= K && ldb >= K && lda % 16 == 0 && ldb % 16 == 0, DF_ERR_ALIGN,
             "%s: lda=%d ldb=%d must be multiples of 16 and >= K=%d", fn, lda, ldb, K);
    DF_CHECK(aligned16(A) && aligned16(B), DF_ERR_ALIGN, "%s: A and B must be 16-byte aligned", fn);
    DF_CHECK(!ws || aligned16(ws), DF_ERR_ALIGN, "%s: workspace must be 16-byte aligned", fn);
    // K is rounded up to the 16-byte granule: the operand rows are zero
    // there (df_quantize_2d pads ld with zeros), so the products vanish.
    g = GemmArgs{A, lda, B, ldb, M, N, (K + 15) & ~15, scale_a_dev, scale_b_dev, bias, C, ldc,
                 static_cast<float*>(ws), ws ? ws_bytes : 0, as_stream(stream)};
    return DF_OK;
}

extern "C" int df_fp8_gemm_nt(int fmt_a, const uint8_t* A, int lda, int fmt_b, const uint8_t* B,
                              int ldb, int M, int N, int K, const float* scale_a_dev,
                              const float* scale_b_dev, int bias_dtype, const void* bias,
                              int c_dtype, void* C, int ldc, void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    GemmArgs g;
    bool empty = false;
    const int st = nt_args("df_fp8_gemm_nt", fmt_a, A, lda, fmt_b, B, ldb, M, N, K, scale_a_dev, scale_b_dev,
                           bias_dtype, bias, c_dtype, C, ldc, ws, ws_bytes, stream, g, empty);
    if (st != DF_OK || empty) return st;
    if (fmt_a == E4M3 && fmt_b == E4M3) dispatch_out<E4M3, E4M3>(g, bias_dtype, c_dtype);
    else if (fmt_a == E5M2 && fmt_b == E4M3) dispatch_out<E5M2, E4M3>(g, bias_dtype, c_dtype);
    else if (fmt_a == E4M3 && fmt_b == E5M2) dispatch_out<E4M3, E5M2>(g, bias_dtype, c_dtype);
    else dispatch_out<E5M2, E5M2>(g, bias_dtype, c_dtype);
    return launch_status("df_fp8_gemm_nt");
}

extern "C" int df_fp8_gemm_nt_plan(int M, int N, int K, int lda, int ldb, const void* bias, size_t ws_bytes,
                                   int* kernel, int* split) {
    clear_error();
    DF_CHECK(kernel && split, DF_ERR_INVALID, "df_fp8_gemm_nt_plan: NULL output");
    DF_CHECK(M > 0 && N > 0 && K > 0, DF_ERR_INVALID, "df_fp8_gemm_nt_plan: sizes must be positive (M=%d N=%d K=%d)",
             M, N, K);
    DF_CHECK(lda >= K && ldb >= K && lda % 16 == 0 && ldb % 16 == 0, DF_ERR_ALIGN,
             "df_fp8_gemm_nt_plan: lda=%d ldb=%d must be multiples of 16 and >= K=%d", lda, ldb, K);
    // the pointers only matter through their alignment (bias) and presence (ws)
    GemmArgs g{nullptr, lda, nullptr, ldb, M, N, (K + 15) & ~15, nullptr, nullptr, bias, nullptr, N,
               ws_bytes ? reinterpret_cast<float*>(uintptr_t{16}) : nullptr, ws_bytes, nullptr};
    const NtPlan p = nt_plan(g);
    *kernel = p.kind;
    *split = p.split;
    return DF_OK;
}

extern "C" int df_fp8_gemm_fwd(const uint8_t* Xq, int ldx, const uint8_t* Wq, int ldw, int M, int N,
                               int K, const float* sx_dev, const float* sw_dev, int bias_dtype,
                               const void* bias, int y_dtype, void* Y, int ldy, void* ws,
                               size_t ws_bytes, void* stream) {
    return df_fp8_gemm_nt(DF_FMT_E4M3, Xq, ldx, DF_FMT_E4M3, Wq, ldw, M, N, K, sx_dev, sw_dev,
                          bias_dtype, bias, y_dtype, Y, ldy, ws, ws_bytes, stream);
}

extern "C" int df_fp8_gemm_fwd_timeline(const uint8_t* Xq, int ldx, const uint8_t* Wq, int ldw, int M, int N, int K,
                                        const float* sx_dev, const float* sw_dev, const uint16_t* bias_bf16,
                                        uint16_t* Y_bf16, int ldy, uint64_t* stamps, int stamps_per_block,
                                        int* grid_out, void* stream) {
    clear_error();
    GemmArgs g;
    bool empty = false;
    const int st = nt_args("df_fp8_gemm_fwd_timeline", DF_FMT_E4M3, Xq, ldx, DF_FMT_E4M3, Wq, ldw, M, N, K, sx_dev,
                           sw_dev, DF_DTYPE_BFLOAT16, bias_bf16, DF_DTYPE_BFLOAT16, Y_bf16, ldy, nullptr, 0, stream, g,
                           empty);
    if (st != DF_OK) return st;
    DF_CHECK(!empty && bias_bf16 && stamps && grid_out && stamps_per_block >= 1, DF_ERR_INVALID,
             "df_fp8_gemm_fwd_timeline: needs M, N > 0, a bias, a stamp buffer and grid_out");
    const NtPlan p = nt_plan(g);
    DF_CHECK(p.kind == DF_GEMM_KERNEL_PERSISTENT && p.split == 1, DF_ERR_UNSUPPORTED,
             "df_fp8_gemm_fwd_timeline: M=%d N=%d K=%d does not run the unsplit 256x256 persistent kernel", M, N, K);
    *grid_out = p.grid;
    gemm_nt_persistent_timeline_kernel<E4M3, E4M3, uint16_t, uint16_t, true><<<p.grid, 512, 0, g.st>>>(
        g.A, g.lda, g.B, g.ldb, g.M, g.N, g.K, g.sa, g.sb, bias_bf16, Y_bf16, g.ldc,
        epi_store_mode(g.C, (int64_t)g.ldc * 2), stamps, stamps_per_block);
    return launch_status("df_fp8_gemm_fwd_timeline");
}

// Forward GEMM whose Y also yields its absmax (and the next quantize's scale):
// the unsplit 256x256 persistent kernel folds |Y| in its epilogue into
// per-block, per-wave partials in ws, and one block folds those.  Other plans
// run df_fp8_gemm_fwd and then df_absmax_scale_* over Y (two passes, the same
// results).
extern "C" size_t df_fp8_gemm_fwd_absmax_workspace_bytes(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    // 8 partials per block; the grid is at most one block per tile
    const size_t parts = (size_t)((M + kPBM - 1) / kPBM) * (size_t)((N + kPBN - 1) / kPBN) * 8 * sizeof(uint32_t);
    return std::max(std::max(parts, df_absmax_workspace_bytes()), df_fp8_gemm_workspace_bytes(M, N, K));
}

extern "C" int df_fp8_gemm_fwd_absmax(const uint8_t* Xq, int ldx, const uint8_t* Wq, int ldw, int M, int N, int K,
                                      const float* sx_dev, const float* sw_dev, int bias_dtype, const void* bias,
                                      int y_dtype, void* Y, int ldy, int next_fmt, float* y_absmax_dev,
                                      float* y_scale_dev, void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    static const char* name = "df_fp8_gemm_fwd_absmax";
    DF_CHECK(y_dtype == DF_DTYPE_BFLOAT16 || y_dtype == DF_DTYPE_HALF || y_dtype == DF_DTYPE_FLOAT32,
             DF_ERR_UNSUPPORTED, "%s: Y dtype %d (bf16, f16 or fp32 only)", name, y_dtype);
    DF_CHECK(next_fmt == E4M3 || next_fmt == E5M2, DF_ERR_UNSUPPORTED, "%s: bad fp8 format %d", name, next_fmt);
    DF_CHECK(y_absmax_dev || y_scale_dev, DF_ERR_INVALID, "%s: no absmax or scale output", name);
    DF_CHECK(ldy == N, DF_ERR_INVALID, "%s: Y must be contiguous (ldy=%d, N=%d)", name, ldy, N);
    GemmArgs g;
    bool empty = false;
    int st = nt_args(name, DF_FMT_E4M3, Xq, ldx, DF_FMT_E4M3, Wq, ldw, M, N, K, sx_dev, sw_dev, bias_dtype, bias,
                     y_dtype, Y, ldy, ws, ws_bytes, stream, g, empty);
    if (st != DF_OK) return st;
    DF_CHECK(ws && ws_bytes >= df_absmax_workspace_bytes(), DF_ERR_WORKSPACE,
             "%s: workspace %zu bytes < %zu", name, ws_bytes, df_absmax_workspace_bytes());
    const bool bf16_out = y_dtype == DF_DTYPE_BFLOAT16, f16_out = y_dtype == DF_DTYPE_HALF;
    const NtPlan p = empty ? NtPlan{} : nt_plan(g);
    if (!empty && p.kind == DF_GEMM_KERNEL_PERSISTENT && p.split == 1 &&
        ws_bytes >= (size_t)p.grid * 8 * sizeof(uint32_t)) {
        uint32_t* parts = static_cast<uint32_t*>(ws);
        const int vec_out = epi_store_mode(g.C, (int64_t)g.ldc * (bf16_out || f16_out ? 2 : 4));
        const bool bbf = bias && bias_dtype == DF_DTYPE_BFLOAT16, bhf = bias && bias_dtype == DF_DTYPE_HALF;
#define DF_AMAX_LAUNCH(OutT, BiasT, HB)                                                                          \
    gemm_nt_persistent_amax_kernel<E4M3, E4M3, OutT, BiasT, HB><<<p.grid, 512, 0, g.st>>>(                      \
        g.A, g.lda, g.B, g.ldb, g.M, g.N, g.K, g.sa, g.sb, static_cast<const BiasT*>(g.bias),                     \
        static_cast<OutT*>(g.C), g.ldc, vec_out, parts)
        if (bf16_out) {
            if (!bias) DF_AMAX_LAUNCH(uint16_t, float, false);
            else if (bbf) DF_AMAX_LAUNCH(uint16_t, uint16_t, true);
            else DF_AMAX_LAUNCH(uint16_t, float, true);
        } else if (f16_out) {  // nt_args admits an fp32 or f16 bias here
            if (!bias) DF_AMAX_LAUNCH(f16_t, float, false);
            else if (bhf) DF_AMAX_LAUNCH(f16_t, f16_t, true);
            else DF_AMAX_LAUNCH(f16_t, float, true);
        } else {
            if (!bias) DF_AMAX_LAUNCH(float, float, false);
            else if (bbf) DF_AMAX_LAUNCH(float, uint16_t, true);
            else DF_AMAX_LAUNCH(float, float, true);
        }
#undef DF_AMAX_LAUNCH
        if ((st = launch_status(name)) != DF_OK) return st;
        // each of the grid's blocks wrote its 8 partials
        launch_absmax_fold(parts, p.grid * 8, next_fmt, y_absmax_dev, y_scale_dev, g.st);
        return launch_status(name);
    }
    st = df_fp8_gemm_fwd(Xq, ldx, Wq, ldw, M, N, K, sx_dev, sw_dev, bias_dtype, bias, y_dtype, Y, ldy, ws, ws_bytes,
                         stream);
    if (st != DF_OK) return st;
    const int64_t n = (int64_t)M * N;
    if (f16_out)
        return df_absmax_scale_f16(static_cast<const uint16_t*>(Y), n, next_fmt, y_absmax_dev, y_scale_dev, ws,
                                   ws_bytes, stream);
    return bf16_out ? df_absmax_scale_bf16(static_cast<const uint16_t*>(Y), n, next_fmt, y_absmax_dev, y_scale_dev,
                                           ws, ws_bytes, stream)
                    : df_absmax_scale_f32(static_cast<const float*>(Y), n, next_fmt, y_absmax_dev, y_scale_dev, ws,
                                          ws_bytes, stream);
}

extern "C" int df_fp8_gemm_bwd_dx(const uint8_t* dYq, int lddy, const uint8_t* Wtq, int ldwt, int M,
                                  int N, int K, const float* sdy_dev, const float* sw_dev,
                                  int dx_dtype, void* dX, int lddx, void* ws, size_t ws_bytes,
                                  void* stream) {
    // dX[M,K] = sum_n dY[m,n] W[n,k]: NT with reduction N, B = W^T [K, N]
    return df_fp8_gemm_nt(DF_FMT_E5M2, dYq, lddy, DF_FMT_E4M3, Wtq, ldwt, M, K, N, sdy_dev, sw_dev,
                          DF_DTYPE_FLOAT32, nullptr, dx_dtype, dX, lddx, ws, ws_bytes, stream);
}

extern "C" int df_fp8_gemm_bwd_dw(const uint8_t* dYtq, int ldyt, const uint8_t* Xtq, int ldxt, int M,
                                  int N, int K, const float* sdy_dev, const float* sx_dev,
                                  int dw_dtype, void* dW, int lddw, void* ws, size_t ws_bytes,
                                  void* stream) {
    // dW[N,K] = sum_m dY[m,n] X[m,k]: NT with reduction M, A = dY^T [N, M], B = X^T [K, M]
    return df_fp8_gemm_nt(DF_FMT_E5M2, dYtq, ldyt, DF_FMT_E4M3, Xtq, ldxt, N, K, M, sdy_dev, sx_dev,
                          DF_DTYPE_FLOAT32, nullptr, dw_dtype, dW, lddw, ws, ws_bytes, stream);
}

// dW [N, K] in NT form: A = dY^T [N, M], B = X^T [K, M], reduction M;
// dX [M, K]: A = dY [M, N], B = W^T [K, N], reduction N.
static void bwd_shapes(int M, int N, int K, GemmArgs& dw, GemmArgs& dx) {
    dw = GemmArgs{};
    dx = GemmArgs{};
    dw.M = N, dw.N = K, dw.K = (M + 15) & ~15;
    dx.M = M, dx.N = K, dx.K = (N + 15) & ~15;
}

extern "C" size_t df_fp8_gemm_bwd_workspace_bytes(int M, int N, int K) {
    size_t need = std::max(df_fp8_gemm_workspace_bytes(M, K, N), df_fp8_gemm_workspace_bytes(N, K, M));
    const int cus = device_cu_count();
    if (cus > 0 && M > 0 && N > 0 && K > 0) {
        GemmArgs dw, dx;
        bwd_shapes(M, N, K, dw, dx);
        const GroupPlan gp = grouped_plan(dw, dx, SIZE_MAX, cus);
        if (gp.grouped && gp.S > 1) need = std::max(need, (size_t)gp.S * (size_t)N * (size_t)K * sizeof(float));
    }
    return need;
}

extern "C" int df_fp8_gemm_bwd_plan(int M, int N, int K, size_t ws_bytes, int* grouped, int* dw_slices) {
    clear_error();
    DF_CHECK(grouped && dw_slices, DF_ERR_INVALID, "df_fp8_gemm_bwd_plan: NULL output");
    *grouped = 0;
    *dw_slices = 0;
    const int cus = device_cu_count();
    if (cus <= 0 || M <= 0 || N <= 0 || K <= 0) return DF_OK;
    GemmArgs dw, dx;
    bwd_shapes(M, N, K, dw, dx);
    const GroupPlan gp = grouped_plan(dw, dx, ws_bytes, cus);
    *grouped = gp.grouped ? 1 : 0;
    *dw_slices = gp.grouped ? gp.S : 0;
    return DF_OK;
}

// df_fp8_gemm_bwd; with amax_part (room for 8 partials per CU), a grouped
// plan also folds |dX| into it and *folded is set.
static int bwd_impl(const uint8_t* dYq, int lddy, const uint8_t* Wtq, int ldwt, const uint8_t* dYtq, int ldyt,
                    const uint8_t* Xtq, int ldxt, int M, int N, int K, const float* sdy_dev, const float* sw_dev,
                    const float* sx_dev, int dx_dtype, void* dX, int lddx, int dw_dtype, void* dW, int lddw,
                    void* ws, size_t ws_bytes, void* stream, uint32_t* amax_part, bool* folded) {
    GemmArgs dx, dw;
    bool ex = false, ew = false;
    int st = nt_args("df_fp8_gemm_bwd (dX)", DF_FMT_E5M2, dYq, lddy, DF_FMT_E4M3, Wtq, ldwt, M, K, N, sdy_dev,
                     sw_dev, DF_DTYPE_FLOAT32, nullptr, dx_dtype, dX, lddx, ws, ws_bytes, stream, dx, ex);
    if (st != DF_OK) return st;
    st = nt_args("df_fp8_gemm_bwd (dW)", DF_FMT_E5M2, dYtq, ldyt, DF_FMT_E4M3, Xtq, ldxt, N, K, M, sdy_dev, sx_dev,
                 DF_DTYPE_FLOAT32, nullptr, dw_dtype, dW, lddw, ws, ws_bytes, stream, dw, ew);
    if (st != DF_OK) return st;
    const int cus = device_cu_count();
    GroupPlan gp{false, 1, 0};
    // grouped launches for fp32/bf16 outputs and for f16 dX with f16 dW;
    // other pairs with f16 take the two separate launches
    const bool h_dx = dx_dtype == DF_DTYPE_HALF, h_dw = dw_dtype == DF_DTYPE_HALF;
    if (!ex && !ew && M > 0 && N > 0 && cus > 0 && persistent_ok(dx) && persistent_ok(dw) && h_dx == h_dw)
        gp = grouped_plan(dw, dx, dw.ws ? dw.ws_bytes : 0, cus);
    if (!gp.grouped) {
        st = df_fp8_gemm_bwd_dx(dYq, lddy, Wtq, ldwt, M, N, K, sdy_dev, sw_dev, dx_dtype, dX, lddx, ws, ws_bytes,
                                stream);
        if (st != DF_OK) return st;
        return df_fp8_gemm_bwd_dw(dYtq, ldyt, Xtq, ldxt, M, N, K, sdy_dev, sx_dev, dw_dtype, dW, lddw, ws, ws_bytes,
                                  stream);
    }
    const bool dw32 = dw_dtype == DF_DTYPE_FLOAT32, dx32 = dx_dtype == DF_DTYPE_FLOAT32;
    if (amax_part) {
        if (h_dx) launch_grouped<f16_t, f16_t>(dw, dx, gp, cus, amax_part);
        else if (dw32 && dx32) launch_grouped<float, float>(dw, dx, gp, cus, amax_part);
        else if (dw32) launch_grouped<float, uint16_t>(dw, dx, gp, cus, amax_part);
        else if (dx32) launch_grouped<uint16_t, float>(dw, dx, gp, cus, amax_part);
        else launch_grouped<uint16_t, uint16_t>(dw, dx, gp, cus, amax_part);
        *folded = true;
    } else if (h_dx) launch_grouped<f16_t, f16_t>(dw, dx, gp, cus);
    else if (dw32 && dx32) launch_grouped<float, float>(dw, dx, gp, cus);
    else if (dw32) launch_grouped<float, uint16_t>(dw, dx, gp, cus);
    else if (dx32) launch_grouped<uint16_t, float>(dw, dx, gp, cus);
    else launch_grouped<uint16_t, uint16_t>(dw, dx, gp, cus);
    return launch_status("df_fp8_gemm_bwd");
}

extern "C" int df_fp8_gemm_bwd(const uint8_t* dYq, int lddy, const uint8_t* Wtq, int ldwt, const uint8_t* dYtq,
                               int ldyt, const uint8_t* Xtq, int ldxt, int M, int N, int K, const float* sdy_dev,
                               const float* sw_dev, const float* sx_dev, int dx_dtype, void* dX, int lddx,
                               int dw_dtype, void* dW, int lddw, void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    return bwd_impl(dYq, lddy, Wtq, ldwt, dYtq, ldyt, Xtq, ldxt, M, N, K, sdy_dev, sw_dev, sx_dev, dx_dtype, dX, lddx,
                    dw_dtype, dW, lddw, ws, ws_bytes, stream, nullptr, nullptr);
}

// The backward whose dX also yields its absmax and the next quantize's
// scale.  The first kBwdAmaxReserve bytes of ws hold the absmax partials
// (8 per block of the grouped launch, one block per CU, or the absmax pass's
// partials); the rest is df_fp8_gemm_bwd's workspace.
constexpr int kBwdAmaxMaxCus = 1024;
constexpr size_t kBwdAmaxReserve = (size_t)kBwdAmaxMaxCus * 8 * sizeof(uint32_t);

extern "C" size_t df_fp8_gemm_bwd_absmax_workspace_bytes(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    return kBwdAmaxReserve + df_fp8_gemm_bwd_workspace_bytes(M, N, K);
}

extern "C" int df_fp8_gemm_bwd_absmax(const uint8_t* dYq, int lddy, const uint8_t* Wtq, int ldwt,
                                      const uint8_t* dYtq, int ldyt, const uint8_t* Xtq, int ldxt, int M, int N,
                                      int K, const float* sdy_dev, const float* sw_dev, const float* sx_dev,
                                      int dx_dtype, void* dX, int lddx, int dw_dtype, void* dW, int lddw,
                                      int next_fmt, float* dx_absmax_dev, float* dx_scale_dev, void* ws,
                                      size_t ws_bytes, void* stream) {
    clear_error();
    static const char* name = "df_fp8_gemm_bwd_absmax";
    DF_CHECK(dx_dtype == DF_DTYPE_BFLOAT16 || dx_dtype == DF_DTYPE_HALF || dx_dtype == DF_DTYPE_FLOAT32,
             DF_ERR_UNSUPPORTED, "%s: dX dtype %d (bf16, f16 or fp32 only)", name, dx_dtype);
    DF_CHECK(next_fmt == E4M3 || next_fmt == E5M2, DF_ERR_UNSUPPORTED, "%s: bad fp8 format %d", name, next_fmt);
    DF_CHECK(dx_absmax_dev || dx_scale_dev, DF_ERR_INVALID, "%s: no absmax or scale output", name);
    DF_CHECK(lddx == K, DF_ERR_INVALID, "%s: dX must be contiguous (lddx=%d, K=%d)", name, lddx, K);
    DF_CHECK(ws && aligned16(ws) && ws_bytes >= kBwdAmaxReserve, DF_ERR_WORKSPACE,
             "%s: needs a 16-byte aligned workspace of at least %zu bytes", name, kBwdAmaxReserve);
    hipStream_t s = as_stream(stream);
    uint32_t* parts = static_cast<uint32_t*>(ws);
    const int cus = device_cu_count();
    bool folded = false;
    int st = bwd_impl(dYq, lddy, Wtq, ldwt, dYtq, ldyt, Xtq, ldxt, M, N, K, sdy_dev, sw_dev, sx_dev, dx_dtype, dX,
                      lddx, dw_dtype, dW, lddw, static_cast<char*>(ws) + kBwdAmaxReserve, ws_bytes - kBwdAmaxReserve,
                      stream, cus > 0 && cus <= kBwdAmaxMaxCus ? parts : nullptr, &folded);
    if (st != DF_OK) return st;
    if (folded) {
        launch_absmax_fold(parts, cus * 8, next_fmt, dx_absmax_dev, dx_scale_dev, s);
        return launch_status(name);
    }
    const int64_t n = (int64_t)M * K;
    if (dx_dtype == DF_DTYPE_HALF)
        return df_absmax_scale_f16(static_cast<const uint16_t*>(dX), n, next_fmt, dx_absmax_dev, dx_scale_dev, ws,
                                   kBwdAmaxReserve, stream);
    return dx_dtype == DF_DTYPE_BFLOAT16
               ? df_absmax_scale_bf16(static_cast<const uint16_t*>(dX), n, next_fmt, dx_absmax_dev, dx_scale_dev,
                                      ws, kBwdAmaxReserve, stream)
               : df_absmax_scale_f32(static_cast<const float*>(dX), n, next_fmt, dx_absmax_dev, dx_scale_dev, ws,
                                     kBwdAmaxReserve, stream);
}
