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

#include "df_common.hpp"

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
__device__ __forceinline__ float bias_ld(const float* b, int i) { return b[i]; }
__device__ __forceinline__ float bias_ld(const uint16_t* b, int i) { return bf16_to_f32(b[i]); }

// 4 consecutive outputs of one row: one 16-byte (fp32) or 8-byte (bf16) store
__device__ __forceinline__ void store4(float* p, const float* v) {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
}
__device__ __forceinline__ void store4(uint16_t* p, const float* v) {
    *reinterpret_cast<u32x2*>(p) = u32x2{f32_to_bf16_rne(v[0]) | (f32_to_bf16_rne(v[1]) << 16),
                                        f32_to_bf16_rne(v[2]) | (f32_to_bf16_rne(v[3]) << 16)};
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

template <int FA, int FB, typename OutT, typename BiasT>
static void launch_shape(const GemmArgs& g) {
    if (plan_gemm(g.M, g.N, g.K, g.ws ? g.ws_bytes : 0).big)
        launch_cfg<256, 256, 2, 4, FA, FB, OutT, BiasT>(g);
    else
        launch_cfg<128, 128, 2, 2, FA, FB, OutT, BiasT>(g);
}

template <int FA, int FB>
static void dispatch_out(const GemmArgs& g, int bias_dtype, int c_dtype) {
    const bool bf16_bias = g.bias && bias_dtype == DF_DTYPE_BFLOAT16;
    if (c_dtype == DF_DTYPE_FLOAT32) {
        if (bf16_bias) launch_shape<FA, FB, float, uint16_t>(g);
        else launch_shape<FA, FB, float, float>(g);
    } else {
        if (bf16_bias) launch_shape<FA, FB, uint16_t, uint16_t>(g);
        else launch_shape<FA, FB, uint16_t, float>(g);
    }
}

}  // namespace dfk

using namespace dfk;

extern "C" size_t df_fp8_gemm_workspace_bytes(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    const int S = plan_split(M, N, (K + 15) & ~15, SIZE_MAX);
    return S > 1 ? (size_t)S * (size_t)M * (size_t)N * sizeof(float) : 0;
}

extern "C" int df_fp8_gemm_nt(int fmt_a, const uint8_t* A, int lda, int fmt_b, const uint8_t* B,
                              int ldb, int M, int N, int K, const float* scale_a_dev,
                              const float* scale_b_dev, int bias_dtype, const void* bias,
                              int c_dtype, void* C, int ldc, void* ws, size_t ws_bytes, void* stream) {
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
    DF_CHECK(!ws || aligned16(ws), DF_ERR_ALIGN, "df_fp8_gemm_nt: workspace must be 16-byte aligned");
    // K is rounded up to the 16-byte granule: the operand rows are zero
    // there (df_quantize_2d pads ld with zeros), so the products vanish.
    GemmArgs g{A, lda, B, ldb, M, N, (K + 15) & ~15, scale_a_dev, scale_b_dev, bias, C, ldc,
               static_cast<float*>(ws), ws ? ws_bytes : 0, as_stream(stream)};
    if (fmt_a == E4M3 && fmt_b == E4M3) dispatch_out<E4M3, E4M3>(g, bias_dtype, c_dtype);
    else if (fmt_a == E5M2 && fmt_b == E4M3) dispatch_out<E5M2, E4M3>(g, bias_dtype, c_dtype);
    else if (fmt_a == E4M3 && fmt_b == E5M2) dispatch_out<E4M3, E5M2>(g, bias_dtype, c_dtype);
    else dispatch_out<E5M2, E5M2>(g, bias_dtype, c_dtype);
    return launch_status("df_fp8_gemm_nt");
}

extern "C" int df_fp8_gemm_fwd(const uint8_t* Xq, int ldx, const uint8_t* Wq, int ldw, int M, int N,
                               int K, const float* sx_dev, const float* sw_dev, int bias_dtype,
                               const void* bias, int y_dtype, void* Y, int ldy, void* ws,
                               size_t ws_bytes, void* stream) {
    return df_fp8_gemm_nt(DF_FMT_E4M3, Xq, ldx, DF_FMT_E4M3, Wq, ldw, M, N, K, sx_dev, sw_dev,
                          bias_dtype, bias, y_dtype, Y, ldy, ws, ws_bytes, stream);
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
