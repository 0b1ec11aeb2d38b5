// Dequant-GEMM on MFMA for the prefill / verify shapes (M >= 64 activation
// rows) on gfx950.
//
// The exact GEMV kernels spend one VALU FMA per weight and activation row, so
// at M >= 64 they would be ~30x slower than the matrix cores.  Here the
// product runs on v_mfma_f32_32x32x16_f16 (fp16 x fp16 -> fp32 accumulate):
//   * weights are unpacked exactly into fp16 integers (int4: -8..7, int8:
//     -128..127) with the exponent-magic trick of the GEMV kernels; for the
//     group formats the fp16 weights of a group are multiplied by the group
//     scale rounded to fp16 (relative error <= 2^-11), per-row scales are
//     applied in fp32 at the end;
//   * activations are converted to fp16 once per tile after scaling each row
//     by a power of two that puts its largest magnitude in [2^14, 2^15): then
//     bf16 -> fp16 is exact for every value within 2^28 of the row's largest,
//     and an fp32 activation becomes two fp16 parts, hi = fp16(a) and
//     lo = fp16(a - hi), multiplied by two MFMAs (22 of its 24 bits survive,
//     so cancelling fp32 activations stay accurate);
//   * group scales are scaled the same way per weight row (largest in
//     [2^11, 2^12), so scale x weight stays below 2^15 and off the fp16
//     subnormals); the epilogue multiplies both powers of two back out, which
//     is exact, so any finite fp32 / bf16 activation and any scale keep the
//     fp16 path's relative accuracy;
//   * products are exact in the MFMA, sums are fp32 in an order that differs
//     from the reference: outputs agree with the reference to ~1e-3 relative
//     (the MFMA path tolerance is 1e-2).
// The weight unpack pairs nibbles (k, k+4) (int4) or bytes (k, k+2) (int8)
// into one fp16x2 register, so every 8-element block of the activation tile is
// stored in the matching order: int4 (0,4,1,5,2,6,3,7), int8 (0,2,1,3,4,6,5,7).
//
// A small pre-pass converts the activations once into that fp16 layout (two
// planes, hi and lo, for fp32 activations) in a per-device scratch buffer.
// W8A16 skips it (BF): v_mfma_f32_32x32x16_bf16 takes the bf16 activations
// as they are, in natural k order, and each int8 weight becomes the bf16 of
// its value (exact: |w| <= 128 has at most 8 significant bits) by one
// sign-extending byte conversion to fp32, two of which one v_perm packs;
// products stay exact and the per-row scale is applied in fp32 at the end.
// Tiling: a workgroup of four waves computes BM x BN outputs (waves WM x WN,
// each (BM/WM) x (BN/WN) in 32 x 32 MFMA tiles) over K in steps of 64, with a
// double-buffered LDS stage filled by global -> LDS DMA (activation blocks
// XOR-swizzled by row, weights row-major, the stage's group scales) while the
// previous step is multiplied; weights are unpacked from LDS into registers
// per 16-k step, and the LDS fragments of the next 16-k step are read while
// the current one is decoded and multiplied.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <mutex>

#include "gemv_device.h"
#include "internal.h"

namespace pilm {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;           // K per stage
constexpr int kMfmaThreads = 256;

template <int FMT>
struct MF {
    static constexpr bool w8 = FMT == F_W8A32 || FMT == F_W8A16;
    static constexpr bool a32 = FMT == F_W8A32;
    static constexpr int group = FMT == F_W4G128 ? 128 : (FMT == F_W4G32 ? 32 : 0);
    static constexpr int wrow = w8 ? kBK : kBK / 2;   // weight bytes per row per stage
    static constexpr int planes = a32 ? 2 : 1;        // fp16 parts per activation
    // chunk swizzle of weight row r in the LDS tile (wrow / 16 chunks per row)
    static __device__ __forceinline__ int wswz(int r) { return w8 ? (r >> 2) & 3 : (r >> 3) & 1; }
};

// fp16 pair of two bf16 values (exact in the fp16 normal range), packed lo/hi.
__device__ __forceinline__ uint32_t f16x2_of_f32(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
}

// Converts one 8-element activation block (k0..k7, as fp32 values) into the
// fp16 order the weight unpack produces, 4 dwords.  (Values that are exact in
// fp16 -- bf16 activations -- may use the truncating pack.)
template <int FMT>
__device__ __forceinline__ u32x4 act_block(const float (&v)[8]) {
    u32x4 o;
    if constexpr (MF<FMT>::w8) {   // (0,2) (1,3) (4,6) (5,7)
        o[0] = f16x2_of_f32(v[0], v[2]);
        o[1] = f16x2_of_f32(v[1], v[3]);
        o[2] = f16x2_of_f32(v[4], v[6]);
        o[3] = f16x2_of_f32(v[5], v[7]);
    } else {                       // (0,4) (1,5) (2,6) (3,7)
        o[0] = f16x2_of_f32(v[0], v[4]);
        o[1] = f16x2_of_f32(v[1], v[5]);
        o[2] = f16x2_of_f32(v[2], v[6]);
        o[3] = f16x2_of_f32(v[3], v[7]);
    }
    return o;
}

// Bytes lo and lo + 1 of u (int8) as a bf16 pair, byte lo in the low half:
// the fp32 of a small integer is exact and its upper 16 bits are its bf16.
__device__ __forceinline__ uint32_t bf16x2_of_i8(uint32_t u, int lo) {
    const float f0 = (float)((int)(u << (24 - 8 * lo)) >> 24);
    const float f1 = (float)((int)(u << (16 - 8 * lo)) >> 24);
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f1), __builtin_bit_cast(uint32_t, f0), 0x07060302u);
}

// fp32 activations: v = hi + lo with hi = fp16(v) (round to nearest) and
// lo = fp16(v - hi); v - hi is exact in fp32.  Overwrites v with lo.
__device__ __forceinline__ void split_hi(float (&v)[8], float (&hi)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float h = (float)(_Float16)v[e];
        hi[e] = h;
        v[e] = (float)(_Float16)(v[e] - h);
    }
}

// Power-of-two exponent e with maxv * 2^e in [2^(top-1), 2^top); 0 for a zero
// or non-finite maximum (such rows convert unscaled, as the reference would
// propagate their infinities and NaNs).
__device__ __forceinline__ int range_exp(float maxv, int top) {
    if (!(maxv > 0.0f) || !__builtin_isfinite(maxv)) return 0;
    int ex;
    (void)frexpf(maxv, &ex);   // maxv in [2^(ex-1), 2^ex)
    return top - ex;
}

__device__ __forceinline__ float block_max_256(float v, float *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

template <int FMT>
__device__ __forceinline__ void load_act8(const void *__restrict__ A, size_t blk, float (&v)[8]) {
    if constexpr (MF<FMT>::a32) {
        const f32x4 *p = (const f32x4 *)A + 2 * blk;
        const f32x4 x0 = p[0], x1 = p[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = x0[e];
            v[4 + e] = x1[e];
        }
    } else {
        const u32x4 x = ((const u32x4 *)A)[blk];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = bf16_lo(x[e]);
            v[2 * e + 1] = bf16_hi(x[e]);
        }
    }
}

// Activations [M, K] (bf16 or fp32) -> X[plane][M][K] fp16, each 8-element
// block in the weight unpack order.  Workgroup m takes activation row m: its
// largest magnitude sets the row exponent E[m], then every value is scaled by
// 2^E[m] (exact) and converted.  The first kPrepHold 8-element blocks of
// each thread stay in registers between the two passes (all of a row up to
// K = 16384), so the row is read once and its loads are issued together.
constexpr int kPrepHold = 8;

template <int FMT>
__global__ __launch_bounds__(256) void act_prep_kernel(const void *__restrict__ A, u32x4 *__restrict__ X,
                                                      int *__restrict__ E, int M, int K) {
    using F = MF<FMT>;
    __shared__ float red[4];
    const int tid = threadIdx.x;
    const int m = blockIdx.x;
    const size_t nb = (size_t)K / 8, row0 = (size_t)m * nb, blocks = (size_t)M * nb;
    float hold[kPrepHold][8];
#pragma unroll
    for (int h = 0; h < kPrepHold; ++h) {
        const size_t b = tid + (size_t)h * 256;
        if (b < nb) load_act8<FMT>(A, row0 + b, hold[h]);
    }
    float mx = 0.0f;
#pragma unroll
    for (int h = 0; h < kPrepHold; ++h) {
        const size_t b = tid + (size_t)h * 256;
        if (b < nb)
#pragma unroll
            for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(hold[h][e]));
    }
    for (size_t b = tid + (size_t)kPrepHold * 256; b < nb; b += 256) {
        float v[8];
        load_act8<FMT>(A, row0 + b, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[e]));
    }
    const int ex = range_exp(block_max_256(mx, red), 15);
    if (tid == 0) E[m] = ex;
    auto put = [&](size_t b, float (&v)[8]) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = ldexpf(v[e], ex);
        if constexpr (F::a32) {
            float hi[8];
            split_hi(v, hi);
            X[row0 + b] = act_block<FMT>(hi);
            X[blocks + row0 + b] = act_block<FMT>(v);
        } else {
            X[row0 + b] = act_block<FMT>(v);
        }
    };
#pragma unroll
    for (int h = 0; h < kPrepHold; ++h) {
        const size_t b = tid + (size_t)h * 256;
        if (b < nb) put(b, hold[h]);
    }
    for (size_t b = tid + (size_t)kPrepHold * 256; b < nb; b += 256) {
        float v[8];
        load_act8<FMT>(A, row0 + b, v);
        put(b, v);
    }
}

// blockIdx.z selects a contiguous range of K steps (split K); with more than
// one split the fp32 sums (the weight-row power of two taken out) go to
// P[z][M][N] and split_reduce_kernel adds them in split order
// (deterministic) and finishes the outputs.
// Group formats scale the group scales of each weight row by a power of two
// 2^wexp that puts the largest scale the workgroup uses in [2^11, 2^12)
// (scale x weight then stays within fp16 and off its subnormals); a
// workgroup finds it from the scales of its own K range, which changes
// nothing but that exact power of two, taken out again in the epilogue.
// X: the activations prepared by act_prep_kernel (fp16, planes x M x K), or
// with BF (W8A16 only) the caller's bf16 activations [M, K] and E unused.
template <int FMT, int BM, int BN, int WM>
constexpr int mfma_stage_bytes() {
    using F = MF<FMT>;
    return BM * kBK * 2 * F::planes + BN * F::wrow + (F::group > 0 ? kMfmaThreads * 4 : 0);
}

// Two resident workgroups per CU where their LDS stages fit (the register
// budget follows), else one.
template <int FMT, int BM, int BN, int WM>
constexpr int mfma_min_blocks() {
    return 4 * mfma_stage_bytes<FMT, BM, BN, WM>() <= 160 * 1024 ? 2 : 1;
}

template <int FMT, int BM, int BN, int WM, bool BF>
__global__ __launch_bounds__(kMfmaThreads, (mfma_min_blocks<FMT, BM, BN, WM>())) void gemm_mfma_kernel(const _Float16 *__restrict__ X,
                                                                const uint8_t *__restrict__ W,
                                                                const float *__restrict__ S, void *__restrict__ C,
                                                                float *__restrict__ P, const int *__restrict__ E,
                                                                int M, int N, int K, int steps_per_split) {
    using F = MF<FMT>;
    static_assert(!BF || FMT == F_W8A16, "bf16 operands: int8 weights with bf16 activations");
    constexpr int WN = 4 / WM;
    constexpr int TM = BM / WM / 32;     // 32x32 tiles per wave along M
    constexpr int TN = BN / WN / 32;     // ... along N
    constexpr int A_PLANE = BM * kBK * 2;
    constexpr int A_BYTES = A_PLANE * F::planes;
    constexpr int W_BYTES = BN * F::wrow;
    constexpr int SPS = F::group == 32 ? 2 : 1;   // groups per stage (group formats)
    // group scales of the stage, one 4-byte DMA per thread: float tid is
    // row tid % BN of the stage's group tid / BN (beyond SPS groups: a copy
    // of the first, unused)
    constexpr int SC_BYTES = F::group > 0 ? kMfmaThreads * 4 : 0;
    constexpr int STAGE = A_BYTES + W_BYTES + SC_BYTES;
    constexpr int A_LOADS = A_PLANE / 16 / kMfmaThreads;     // 16-byte DMA per thread per plane and stage
    constexpr int W_LOADS = W_BYTES / 16 / kMfmaThreads;
    static_assert(A_LOADS >= 1 && W_LOADS >= 1, "tile too small");
    static_assert(F::group == 0 || (kMfmaThreads % BN == 0 && SPS * BN <= kMfmaThreads), "scale slots");
    static_assert(STAGE == mfma_stage_bytes<FMT, BM, BN, WM>(), "stage layout");
    __shared__ __align__(16) unsigned char lds[2 * STAGE];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int wm = wave % WM, wn = wave / WM;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const size_t row_bytes = F::w8 ? (size_t)K : (size_t)K / 2;
    const int t0 = blockIdx.z * steps_per_split;
    const int nsteps = min(steps_per_split, K / kBK - t0);   // >= 1 (host guarantees)
    const size_t plane = (size_t)M * K;

    // Activation tile: row r holds 8 blocks of 16 B; block kb sits at position
    // kb ^ ((r >> 1) & 7) so that 16 lanes reading one block of 16 rows cover
    // all banks.  The DMA writes positions in lane order, so each lane fetches
    // the block that belongs at its position.
    auto load_a = [&](int t, int b) {
        unsigned char *as = lds + b * STAGE;
#pragma unroll
        for (int pl = 0; pl < F::planes; ++pl)
#pragma unroll
            for (int i = 0; i < A_LOADS; ++i) {
                const int c = i * kMfmaThreads + tid;            // 16-byte position in the plane
                const int row = c >> 3, pos = c & 7;
                const int kb = pos ^ ((row >> 1) & 7);
                const int m = min(m0 + row, M - 1);
                const _Float16 *src = X + pl * plane + (size_t)m * K + (size_t)(t0 + t) * kBK + 8 * kb;
                __builtin_amdgcn_global_load_lds((const void *)src,
                                                 (lds_void *)(as + pl * A_PLANE + (i * kMfmaThreads + wave * 64) * 16),
                                                 16, 0, 0);
            }
    };
    // Weight tile: wrow bytes per row, by DMA (16 B per lane); the row's
    // 16-byte chunks sit at positions ch ^ wswz(row), so that the 32 rows a
    // wave reads at one k fall on different LDS banks (rows 8 apart for int4,
    // 4 apart for int8 would otherwise share them).
    auto load_w = [&](int t, int b) {
        unsigned char *ws = lds + b * STAGE + A_BYTES;
#pragma unroll
        for (int i = 0; i < W_LOADS; ++i) {
            const int idx = tid + i * kMfmaThreads;            // 16-byte position in the tile
            const int row = idx / (F::wrow / 16), pos = idx % (F::wrow / 16);
            const int ch = pos ^ F::wswz(row);
            const int n = min(n0 + row, N - 1);
            const uint8_t *src = W + (size_t)n * row_bytes + (size_t)(t0 + t) * F::wrow + ch * 16;
            __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)(ws + (i * kMfmaThreads + wave * 64) * 16),
                                             16, 0, 0);
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x16{};

    const int mrow_base = wm * (BM / WM);
    const int ncol_base = wn * (BN / WN);
    const int G = F::group > 0 ? (K + F::group - 1) / F::group : 1;
    auto load_sc = [&](int t, int b) {
        if constexpr (F::group > 0) {
            const int gl = tid / BN, row = tid % BN;
            const int g = min(((t0 + t) * kBK) / F::group + (gl < SPS ? gl : 0), G - 1);
            const float *src = S + (size_t)min(n0 + row, N - 1) * G + g;
            __builtin_amdgcn_global_load_lds((const void *)src,
                                             (lds_void *)(lds + b * STAGE + A_BYTES + W_BYTES + wave * 256), 4, 0, 0);
        }
    };
    auto issue = [&](int t, int b) {
        load_a(t, b);
        load_w(t, b);
        load_sc(t, b);
    };

    issue(0, 0);
    // weight-row exponents (group formats): scales are taken times 2^wexp;
    // the scale loads overlap the first stage's DMA
    int wexp[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        wexp[j] = 0;
        if constexpr (F::group > 0) {
            const int n = min(n0 + ncol_base + j * 32 + (lane & 31), N - 1);
            const int g0 = (t0 * kBK) / F::group, g1 = min(G, ((t0 + nsteps) * kBK + F::group - 1) / F::group);
            const float *sr = S + (size_t)n * G;
            float mx = 0.0f;
#pragma unroll 16
            for (int g = g0; g < g1; ++g) mx = fmaxf(mx, fabsf(sr[g]));
            wexp[j] = range_exp(mx, 12);
        }
    }
    wait_vmcnt<0>();
    __syncthreads();

    const uint32_t magic = opaque_magic();
    for (int t = 0; t < nsteps; ++t) {
        const int b = t & 1;
        if (t + 1 < nsteps) issue(t + 1, b ^ 1);
        const unsigned char *as = lds + b * STAGE;
        const unsigned char *ws = as + A_BYTES;
        h2 spair[TN][SPS];
        if constexpr (F::group > 0) {
            const float *scs = (const float *)(ws + W_BYTES);
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int g = 0; g < SPS; ++g) {
                    const _Float16 h = (_Float16)ldexpf(scs[g * BN + ncol_base + j * 32 + (lane & 31)], wexp[j]);
                    spair[j][g] = h2{h, h};
                }
        }
        // LDS fragments of step kk + 1 are read while step kk decodes and
        // multiplies (raw weight words and activation blocks, two slots)
        uint32_t wraw[2][TN][F::w8 ? 2 : 1];
        half8 afr[2][TM][F::planes];
        auto read_frags = [&](int kk, int slot) {
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int nl = ncol_base + j * 32 + (lane & 31);
                if constexpr (F::w8) {
                    // bytes k..k+7 of row nl: k = 16 kk + 8 (lane >> 5), chunk kk
                    const uint32_t *pw =
                        (const uint32_t *)(ws + nl * F::wrow + ((kk ^ F::wswz(nl)) << 4) + 8 * (lane >> 5));
                    wraw[slot][j][0] = pw[0];
                    wraw[slot][j][F::w8 ? 1 : 0] = pw[1];
                } else {
                    // nibbles k..k+7 of row nl: byte 8 kk + 4 (lane >> 5), chunk kk / 2
                    wraw[slot][j][0] = *(const uint32_t *)(ws + nl * F::wrow + (((kk >> 1) ^ F::wswz(nl)) << 4) +
                                                           8 * (kk & 1) + 4 * (lane >> 5));
                }
            }
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int row = mrow_base + i * 32 + (lane & 31);
                const int kb = 2 * kk + (lane >> 5);
#pragma unroll
                for (int pl = 0; pl < F::planes; ++pl)
                    afr[slot][i][pl] =
                        *(const half8 *)(as + pl * A_PLANE + row * (kBK * 2) + ((kb ^ ((row >> 1) & 7)) << 4));
            }
        };
        read_frags(0, 0);
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            const int slot = kk & 1;
            if (kk + 1 < kBK / 16) read_frags(kk + 1, slot ^ 1);
            __builtin_amdgcn_sched_barrier(0);   // keep those reads ahead of this step's work
            half8 bfr[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                u32x4 q;
                if constexpr (BF) {   // natural order: (0,1) (2,3) (4,5) (6,7)
#pragma unroll
                    for (int d = 0; d < 2; ++d) {
                        q[2 * d] = bf16x2_of_i8(wraw[slot][j][d], 0);
                        q[2 * d + 1] = bf16x2_of_i8(wraw[slot][j][d], 2);
                    }
                } else if constexpr (F::w8) {
                    const h2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
#pragma unroll
                    for (int d = 0; d < 2; ++d) {
                        const uint32_t u = wraw[slot][j][F::w8 ? d : 0] ^ 0x80808080u;
                        const h2 lo = __builtin_bit_cast(h2, (u & 0x00FF00FFu) | magic) + bias;
                        const h2 hi = __builtin_bit_cast(h2, ((u >> 8) & 0x00FF00FFu) | magic) + bias;
                        q[2 * d] = __builtin_bit_cast(uint32_t, lo);
                        q[2 * d + 1] = __builtin_bit_cast(uint32_t, hi);
                    }
                } else {
                    h2 qq[4];
                    dequant_w4(wraw[slot][j][0], magic, qq);
                    if constexpr (F::group > 0) {
                        const h2 sp = spair[j][SPS == 2 ? (kk >> 1) : 0];
#pragma unroll
                        for (int e = 0; e < 4; ++e) qq[e] = qq[e] * sp;
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e) q[e] = __builtin_bit_cast(uint32_t, qq[e]);
                }
                bfr[j] = __builtin_bit_cast(half8, q);
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int pl = 0; pl < F::planes; ++pl)
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        if constexpr (BF)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                                __builtin_bit_cast(bf16x8, afr[slot][i][pl]), __builtin_bit_cast(bf16x8, bfr[j]),
                                acc[i][j], 0, 0, 0);
                        else
                            acc[i][j] =
                                __builtin_amdgcn_mfma_f32_32x32x16_f16(afr[slot][i][pl], bfr[j], acc[i][j], 0, 0, 0);
                    }
        }
        wait_vmcnt<0>();               // stage t + 1 has landed
        __syncthreads();               // ... and stage t's buffer is free for stage t + 2
    }

    // ---- epilogue: lane holds column (lane & 31) of each tile, rows
    // 8q + 4 (lane >> 5) + r for element 4q + r.
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = n0 + ncol_base + j * 32 + (lane & 31);
        if (n >= N) continue;
        const float sc = (F::group > 0 || P) ? 1.0f : S[n];
        float *pz = P ? P + (size_t)blockIdx.z * M * N : nullptr;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + mrow_base + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (m >= M) continue;
                if (pz) {
                    pz[(size_t)m * N + n] = ldexpf(acc[i][j][e], -wexp[j]);
                    continue;
                }
                const float y = ldexpf(acc[i][j][e], -((BF ? 0 : E[m]) + wexp[j])) * sc;
                if constexpr (F::a32)
                    ((float *)C)[(size_t)m * N + n] = y;
                else
                    ((uint16_t *)C)[(size_t)m * N + n] = f32_to_bf16(y);
            }
    }
}

// Sum of the split partials in split order, then the per-row scale (per-row
// formats) and the output conversion.
template <int FMT>
__global__ __launch_bounds__(256) void split_reduce_kernel(const float *__restrict__ P, const float *__restrict__ S,
                                                          void *__restrict__ C, const int *__restrict__ E, int M,
                                                          int N, int splits) {
    using F = MF<FMT>;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t total = (size_t)M * N;
    if (idx >= total) return;
    float y = 0.0f;
    for (int z = 0; z < splits; ++z) y += P[(size_t)z * total + idx];
    const int m = (int)(idx / N), n = (int)(idx % N);
    if (E) y = ldexpf(y, -E[m]);   // null: activations taken unscaled (BF)
    if constexpr (F::group == 0) y *= S[n];
    if constexpr (F::a32)
        ((float *)C)[idx] = y;
    else
        ((uint16_t *)C)[idx] = f32_to_bf16(y);
}

template <int FMT, int BM, int BN, int WM, bool BF = false>
void launch_mfma(hipStream_t st, const _Float16 *X, const uint8_t *W, const float *S, void *C, float *P,
                 const int *E, int splits, int sps, int M, int N, int K) {
    const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM), (unsigned)splits);
    gemm_mfma_kernel<FMT, BM, BN, WM, BF><<<grid, kMfmaThreads, 0, st>>>(X, W, S, C, splits > 1 ? P : nullptr, E, M,
                                                                         N, K, sps);
    if (splits > 1) {
        const size_t total = (size_t)M * N;
        split_reduce_kernel<FMT><<<(unsigned)((total + 255) / 256), 256, 0, st>>>(P, S, C, E, M, N, splits);
    }
}

// Output tile per workgroup: bm x 128 (bm chosen by run_mfma; 64, 128 or
// 256), waves 1 x 4 for int4 weights and 2 x 2 for int8 (PILM_HIP_MFMA_WM
// overrides).
template <int FMT>
void launch_mfma_fmt(int bm, hipStream_t st, const void *A, const _Float16 *X, int *E, const uint8_t *W,
                     const float *S, void *C, float *P, int splits, int sps, int M, int N, int K) {
    act_prep_kernel<FMT><<<(unsigned)M, 256, 0, st>>>(A, (u32x4 *)X, E, M, K);
    // waves 1 x 4 (each wave all of the tile's rows, a quarter of its
    // columns, so every weight is decoded once) for int4 weights: 8B gate_up
    // W4 g128 M = 64 47.9 vs 53.2 us, M = 80 59.8 vs 71.1 us, M = 1024 261 vs
    // 282 us, M = 2048 (128-row tiles) 504 vs 548 us; 2 x 2 for int8 (its
    // cheaper decode gains nothing from it: W8A32 gate_up M = 1024 443 vs 445 us)
    int wm = MF<FMT>::w8 ? 2 : 1;
    const int env_wm = env_int("PILM_HIP_MFMA_WM", 0);
    if (env_wm == 1 || env_wm == 2) wm = env_wm;
    if (bm == 256)
        wm == 1 ? launch_mfma<FMT, 256, 128, 1>(st, X, W, S, C, P, E, splits, sps, M, N, K)
                : launch_mfma<FMT, 256, 128, 2>(st, X, W, S, C, P, E, splits, sps, M, N, K);
    else if (bm == 128)
        wm == 1 ? launch_mfma<FMT, 128, 128, 1>(st, X, W, S, C, P, E, splits, sps, M, N, K)
                : launch_mfma<FMT, 128, 128, 2>(st, X, W, S, C, P, E, splits, sps, M, N, K);
    else
        wm == 1 ? launch_mfma<FMT, 64, 128, 1>(st, X, W, S, C, P, E, splits, sps, M, N, K)
                : launch_mfma<FMT, 64, 128, 2>(st, X, W, S, C, P, E, splits, sps, M, N, K);
}

// W8A16 on bf16 MFMAs: no activation pass, the kernel reads A directly.
void launch_mfma_bf16(int bm, hipStream_t st, const void *A, const uint8_t *W, const float *S, void *C, float *P,
                      int splits, int sps, int M, int N, int K) {
    const _Float16 *X = (const _Float16 *)A;   // bf16 [M, K]; only copied by byte
    int wm = 2;
    const int env_wm = env_int("PILM_HIP_MFMA_WM", 0);
    if (env_wm == 1 || env_wm == 2) wm = env_wm;
    if (bm == 256)
        wm == 1 ? launch_mfma<F_W8A16, 256, 128, 1, true>(st, X, W, S, C, P, nullptr, splits, sps, M, N, K)
                : launch_mfma<F_W8A16, 256, 128, 2, true>(st, X, W, S, C, P, nullptr, splits, sps, M, N, K);
    else if (bm == 128)
        wm == 1 ? launch_mfma<F_W8A16, 128, 128, 1, true>(st, X, W, S, C, P, nullptr, splits, sps, M, N, K)
                : launch_mfma<F_W8A16, 128, 128, 2, true>(st, X, W, S, C, P, nullptr, splits, sps, M, N, K);
    else
        wm == 1 ? launch_mfma<F_W8A16, 64, 128, 1, true>(st, X, W, S, C, P, nullptr, splits, sps, M, N, K)
                : launch_mfma<F_W8A16, 64, 128, 2, true>(st, X, W, S, C, P, nullptr, splits, sps, M, N, K);
}

}  // namespace

// Row threshold of the matrix-core path: ecpu_hip_set_matrix_core_min_rows()
// when set (>= 0), else PILM_HIP_MFMA_MIN_M, default 64.
static std::atomic<int> g_mfma_min_rows{-1};

int mfma_min_m() {
    const int v = g_mfma_min_rows.load(std::memory_order_relaxed);
    return v >= 0 ? v : env_int("PILM_HIP_MFMA_MIN_M", 64);
}

bool mfma_supports(size_t K, const void *A, const uint8_t *W) {
    return K > 0 && K % kBK == 0 && ((((uintptr_t)A) | ((uintptr_t)W)) & 15) == 0;
}

// Shapes that mfma_supports(); M, N, K below 2^31 (checked by the caller).
int run_mfma(int fmt, size_t M, size_t N, size_t K, const void *A, const uint8_t *W, const float *S, void *C,
             hipStream_t st, const char *fn) {
    if (!mfma_supports(K, A, W)) return fail(ECPU_ERR_UNSUPPORTED, "%s: shape not taken by the matrix-core path", fn);
    // 128-row tiles from M = 128, 64 below; int4 weights take 256-row tiles
    // where the grid still gives every CU two workgroups (each wave then
    // multiplies every decoded weight by 256 rows: 8B W4 g128 gate_up M = 2048
    // 475 vs 504 us, q_proj 174 vs 185 us; with fewer tiles, down M = 2048 and
    // q_proj M = 1024, the 128-row tiles win: 277 vs 291 us, 103 vs 130 us).
    // W8A32's two activation planes leave one 256-row workgroup per CU
    // (gate_up M = 2048 959 vs 894 us).
    int bm = M >= 128 ? 128 : 64;
    const bool w4 = fmt == F_W4ROW || fmt == F_W4G128 || fmt == F_W4G32;
    if (w4 && M >= 256 && ((N + 127) / 128) * ((M + 255) / 256) >= 512) bm = 256;
    const int env_bm = env_int("PILM_HIP_MFMA_BM", 0);
    if (env_bm == 64 || env_bm == 128 || env_bm == 256) bm = env_bm;
    const size_t blocks = ((N + 127) / 128) * ((M + bm - 1) / bm);
    const int nsteps = (int)(K / kBK);
    // Split K while the output tiles alone leave CUs idle: aim at ~256
    // workgroups, each keeping at least four K steps.  More splits cost more
    // than they fill: every split writes and the reduction reads an M x N fp32
    // partial (at M = 64, 32 splits of o_proj move 4x its weight bytes).
    // Measured best split counts land at 256 workgroups (8B W4 g128 M = 64:
    // o_proj 30.5 -> 21.3 us, gate_up 55.1 -> 44.7, down 39.4 -> 32.6, k_proj
    // 22.1 -> 17.5; M = 256: o_proj 43.8 -> 32.3, gate_up 107 -> 92).
    int splits = 1;
    if (blocks < 256)
        splits = (int)std::min<size_t>((size_t)std::max(1, nsteps / 4), (256 + blocks - 1) / blocks);
    const int env_splits = env_int("PILM_HIP_MFMA_SPLITS", 0);
    if (env_splits > 0) splits = std::min(env_splits, nsteps);
    const int sps = (nsteps + splits - 1) / splits;
    splits = (nsteps + sps - 1) / sps;   // every split non-empty
    float *P = nullptr;
    if (splits > 1) {
        int *T = nullptr;
        const int rc = split_scratch(st, (size_t)splits * M * N, 1, &P, &T, fn);
        if (rc != ECPU_OK) return rc;
    }
    // W8A16 runs on bf16 MFMAs straight from the caller's activations
    // (PILM_HIP_MFMA_BF16=0: the fp16 path with its activation pass)
    if (fmt == F_W8A16 && env_int("PILM_HIP_MFMA_BF16", 1) != 0) {
        launch_mfma_bf16(bm, st, A, W, S, C, P, splits, sps, (int)M, (int)N, (int)K);
        return ECPU_OK;
    }
    // activation planes, then the activation-row exponents
    void *X = nullptr;
    const size_t xbytes = ((size_t)M * K * 2 * (fmt == F_W8A32 ? 2 : 1) + 255) & ~(size_t)255;
    {
        const int rc = act_scratch(xbytes + M * sizeof(int), &X, fn);
        if (rc != ECPU_OK) return rc;
    }
    const _Float16 *Xh = (const _Float16 *)X;
    int *E = (int *)((char *)X + xbytes);
    switch (fmt) {
        case F_W8A32: launch_mfma_fmt<F_W8A32>(bm, st, A, Xh, E, W, S, C, P, splits, sps, (int)M, (int)N, (int)K); break;
        case F_W8A16: launch_mfma_fmt<F_W8A16>(bm, st, A, Xh, E, W, S, C, P, splits, sps, (int)M, (int)N, (int)K); break;
        case F_W4ROW: launch_mfma_fmt<F_W4ROW>(bm, st, A, Xh, E, W, S, C, P, splits, sps, (int)M, (int)N, (int)K); break;
        case F_W4G128: launch_mfma_fmt<F_W4G128>(bm, st, A, Xh, E, W, S, C, P, splits, sps, (int)M, (int)N, (int)K); break;
        default: launch_mfma_fmt<F_W4G32>(bm, st, A, Xh, E, W, S, C, P, splits, sps, (int)M, (int)N, (int)K); break;
    }
    return ECPU_OK;
}

}  // namespace pilm

extern "C" int ecpu_hip_set_matrix_core_min_rows(int rows) {
    pilm::g_mfma_min_rows.store(rows < 0 ? -1 : rows, std::memory_order_relaxed);
    return ECPU_OK;
}

extern "C" int ecpu_hip_matrix_core_min_rows(void) { return pilm::mfma_min_m(); }
