// Exact quantized GEMV / small-M GEMM for gfx950.
//
// "Exact" means bit-identical to the reference CPU kernels: every output is
// produced by the same sequence of fp32 roundings as in
//   src/ecpu/src/kernel/kernels.c:78-109, 330-393   (int8: 8 FMA lanes, lane l
//        owns k = l mod 8, hsum ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)), FMA tail)
//   src/ecpu/src/kernel/kernels.c:111-225           (int4: lanes lo[l] take
//        k = 16c+l, hi[l] take 16c+8+l, hsum(lo+hi), FMA tail in pairs)
//   src/ecpu/src/kernel/kernels.c:1089-1139         (groups: fresh int4 dot per
//        group, acc = fma(block, scale[g], acc) in group order)
// followed by the reference's final multiply / bf16 rounding.  An FMA chain
// cannot be split without changing its roundings, so the parallelism is laid
// out around the chains rather than across them:
//
//   * one lane owns one output row (all of that row's chains live in its
//     registers); a wave covers a tile of 64 consecutive rows;
//   * the wave streams its rows in 128-byte stripes (one cache line per row)
//     that a global -> LDS DMA lands XOR-swizzled in an 8 KB slot, from where
//     every lane reads its own row conflict-free;
//   * activations are the same for all lanes of a wave (same k), so they
//     arrive through scalar loads and feed v_fma_mix_f32 / v_fma_f32 as SGPR
//     operands;
//   * int4 nibbles become exact fp16 values with one and-or against the 1024
//     exponent pattern plus one packed fp16 add (or fma) per nibble pair;
//     v_fma_mix_f32 then performs fma(a, w, acc) with w widened exactly;
//   * group-scaled formats may divide K among several waves: the per-group
//     block sums meet in LDS (waves of one workgroup) or in global memory
//     (several workgroups), and one lane per row folds them with the scales
//     in group order (the only serial part of the group formula).
//
// Shapes the stripe loop cannot take (K not a multiple of the stripe,
// unaligned pointers) run a one-thread-per-output kernel that follows the
// reference loops literally, tails included.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "gemv_device.h"
#include "internal.h"

namespace pilm {

// Shape and launch geometry; the buffers travel as separate __restrict__
// kernel arguments so the compiler can prove the activations are never
// written and fetch them with scalar loads.
struct GemvArgs {
    const void *A;
    const uint8_t *W;
    const float *S;
    void *C;
    float *P;                // per-group block sums when K is split
    int *T;                  // per-tile tickets (zero between launches)
    int M, N, K;
    int row_bytes;           // bytes per weight row
    int nstripes;            // 128-byte stripes per row (fast path)
    int sps;                 // stripes per part
    int pl;                  // parts of a tile inside one workgroup (one wave each)
    int pg;                  // workgroups per tile (group formats; block sums meet in global memory)
    int ntiles;              // ceil(N / 64)
    int G;                   // scale groups per row (group formats)
    int scale_slot_bytes;    // LDS per wave for the scales of one stripe
};

// One 16-element chunk of the int4 dot for MT activation rows: lo lanes get
// k0..k0+7 (dword xl), hi lanes get k0+8..k0+15 (dword xh).  act[m][0..7]
// hold the chunk's 16 bf16 activations of row m as 8 dwords.
template <int MT, int STRIDE>
__device__ __forceinline__ void w4_chunk(uint32_t xl, uint32_t xh, const uint32_t *act, uint32_t magic,
                                         float (&lo)[MT][8], float (&hi)[MT][8]) {
    h2 ql[4], qh[4];
    dequant_w4(xl, magic, ql);
    dequant_w4(xh, magic, qh);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const uint32_t *a = act + m * STRIDE;
        lo[m][0] = __builtin_fmaf(bf16_lo(a[0]), (float)ql[0].x, lo[m][0]);
        lo[m][1] = __builtin_fmaf(bf16_hi(a[0]), (float)ql[1].x, lo[m][1]);
        lo[m][2] = __builtin_fmaf(bf16_lo(a[1]), (float)ql[2].x, lo[m][2]);
        lo[m][3] = __builtin_fmaf(bf16_hi(a[1]), (float)ql[3].x, lo[m][3]);
        lo[m][4] = __builtin_fmaf(bf16_lo(a[2]), (float)ql[0].y, lo[m][4]);
        lo[m][5] = __builtin_fmaf(bf16_hi(a[2]), (float)ql[1].y, lo[m][5]);
        lo[m][6] = __builtin_fmaf(bf16_lo(a[3]), (float)ql[2].y, lo[m][6]);
        lo[m][7] = __builtin_fmaf(bf16_hi(a[3]), (float)ql[3].y, lo[m][7]);
        hi[m][0] = __builtin_fmaf(bf16_lo(a[4]), (float)qh[0].x, hi[m][0]);
        hi[m][1] = __builtin_fmaf(bf16_hi(a[4]), (float)qh[1].x, hi[m][1]);
        hi[m][2] = __builtin_fmaf(bf16_lo(a[5]), (float)qh[2].x, hi[m][2]);
        hi[m][3] = __builtin_fmaf(bf16_hi(a[5]), (float)qh[3].x, hi[m][3]);
        hi[m][4] = __builtin_fmaf(bf16_lo(a[6]), (float)qh[0].y, hi[m][4]);
        hi[m][5] = __builtin_fmaf(bf16_hi(a[6]), (float)qh[1].y, hi[m][5]);
        hi[m][6] = __builtin_fmaf(bf16_lo(a[7]), (float)qh[2].y, hi[m][6]);
        hi[m][7] = __builtin_fmaf(bf16_hi(a[7]), (float)qh[3].y, hi[m][7]);
    }
}

__device__ __forceinline__ float w4_block_and_reset(float (&lo)[8], float (&hi)[8]) {
    float s[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) {
        s[l] = lo[l] + hi[l];
        lo[l] = 0.0f;
        hi[l] = 0.0f;
    }
    return hsum8(s);
}

constexpr int kLoads = 8;           // 16-byte DMA loads per lane per stripe (64 rows x 128 B)
constexpr int kMaxParts = 8;        // waves (K parts of one tile) per workgroup, at most
constexpr int kSlotBytes = 64 * kLoads * 16;   // one stripe: 64 rows x 128 B

template <int FMT>
struct StripeFmt {
    static constexpr bool w8 = (FMT == F_W8A32 || FMT == F_W8A16);
    static constexpr bool group = (FMT == F_W4G128 || FMT == F_W4G32);
    static constexpr int k_per_stripe = w8 ? kStripe : 2 * kStripe;               // 128 or 256
    static constexpr int groups_per_stripe = FMT == F_W4G128 ? 2 : (FMT == F_W4G32 ? 8 : 0);
    static constexpr int scale_words = FMT == F_W4G32 ? 8 : (FMT == F_W4G128 ? 2 : 1);
};

// Issues the DMA loads of stripe `st` into the wave's LDS slot: kLoads
// 16-byte weight loads per lane (non-temporal), plus the lane's group scales
// for the stripe when the wave folds the groups itself (two 4-byte loads for
// g128, two 16-byte loads for g32; each lands lane-linear in scale_slot).
template <int FMT>
__device__ __forceinline__ void issue_stripe(const uint8_t *const (&src)[kLoads], const float *ssrc, int st,
                                             bool scale_dma, u32x4 *slot, float *scale_slot) {
    using F = StripeFmt<FMT>;
#pragma unroll
    for (int i = 0; i < kLoads; ++i)
        __builtin_amdgcn_global_load_lds((const void *)(src[i] + (size_t)st * kStripe), (lds_void *)(slot + 64 * i), 16,
                                         0, kNT);
    if constexpr (F::group) {
        if (scale_dma) {
            // (the DMA size is a literal in each branch: the host compilation
            // pass rejects target-dependent sizes of this builtin)
            const float *sp = ssrc + (size_t)st * F::groups_per_stripe;
            if constexpr (FMT == F_W4G32) {
                __builtin_amdgcn_global_load_lds((const void *)sp, (lds_void *)scale_slot, 16, 0, 0);
                __builtin_amdgcn_global_load_lds((const void *)(sp + 4), (lds_void *)(scale_slot + 256), 16, 0, 0);
            } else {
                __builtin_amdgcn_global_load_lds((const void *)sp, (lds_void *)scale_slot, 4, 0, 0);
                __builtin_amdgcn_global_load_lds((const void *)(sp + 1), (lds_void *)(scale_slot + 64), 4, 0, 0);
            }
        }
    }
}

// Stripe-streaming exact kernel.
//
// A wave owns a tile of 64 consecutive rows (lane = row) and a contiguous
// range of that tile's 128-byte stripes.  The stripes of a tile are divided
// into p.pl parts inside one workgroup (one wave per part) and, for group
// formats only, into p.pg workgroups:
//   * pg == 1: part 0 folds its own groups as it goes; parts 1.. leave their
//     per-group block sums (and scales) in LDS, and after a barrier part 0
//     continues the fold with them in group order;
//   * pg > 1: every part stores its block sums to global memory, and the last
//     wave of the tile to arrive folds all of them in group order.
// Per-row formats keep one part per tile (their FMA chains run over all K).
//
// Each wave streams its stripes (64 rows x 128 B) through one 8 KB LDS slot
// filled by global_load_lds_dwordx4 (global -> LDS without VGPRs,
// non-temporal): the wave waits for stripe s, copies it to registers,
// refills the slot with stripe s + 1 and computes stripe s meanwhile.
// Lane t of DMA instruction i fetches row 8i + t/8, 16-byte chunk
// (t & 7) ^ ((row >> 1) & 7): the eight lanes of a row cover its full line,
// and the data lands XOR-swizzled so that lane r reading its own row is
// free of LDS bank conflicts.
//
// Dynamic LDS: pl slots of kSlotBytes, pl scale slots of p.scale_slot_bytes,
// then (pg == 1, pl > 1) the fold area: float blocks[G - G0][MT][64] followed
// by float scales[G - G0][64], where G0 = groups of part 0.
template <int FMT, int MT>
__global__ __launch_bounds__(64 * kMaxParts) void gemv_exact_kernel(const void *__restrict__ A_,
                                                                   const uint8_t *__restrict__ W_,
                                                                   const float *__restrict__ S_, void *__restrict__ C_,
                                                                   float *__restrict__ P_, int *__restrict__ T_,
                                                                   GemvArgs p, int m0) {
    p.A = A_;
    p.W = W_;
    p.S = S_;
    p.C = C_;
    p.P = P_;
    p.T = T_;
    using F = StripeFmt<FMT>;
    extern __shared__ __align__(16) unsigned char lds[];
    // threadIdx.x >> 6 is the same for all lanes of a wave; readfirstlane
    // tells the compiler so, which keeps the part indices in SGPRs.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int tile = blockIdx.x / p.pg;
    const int part = (blockIdx.x - tile * p.pg) * p.pl + wave;
    const int nparts = p.pg * p.pl;
    const bool global_split = F::group && p.pg > 1;
    const bool local_split = F::group && !global_split && p.pl > 1;
    const int row0 = tile * 64;
    const int n = row0 + lane;
    const int nc = n < p.N ? n : p.N - 1;
    const int s0 = min(part * p.sps, p.nstripes);
    const int s1 = min(s0 + p.sps, p.nstripes);
    const int G0 = min(p.sps * F::groups_per_stripe, p.G);   // groups of part 0 (local split)

    const uint8_t *src[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int r = 8 * i + (lane >> 3);
        const int q = (lane & 7) ^ ((r >> 1) & 7);
        src[i] = p.W + (size_t)min(row0 + r, p.N - 1) * p.row_bytes + q * 16;
    }
    const int swz = (lane >> 1) & 7;
    // Unless the block sums go to global memory, the lane's group scales ride
    // along with each stripe.
    const bool scale_dma = F::group && !global_split;
    const float *ssrc = p.S + (size_t)nc * p.G;
    u32x4 *my_slot = (u32x4 *)(lds + wave * kSlotBytes);
    float *my_scales = (float *)(lds + p.pl * kSlotBytes + wave * p.scale_slot_bytes);
    float *fold_blocks = (float *)(lds + p.pl * (kSlotBytes + p.scale_slot_bytes));
    float *fold_scales = fold_blocks + (size_t)(p.G - G0) * MT * 64;
    if (s0 < s1) issue_stripe<FMT>(src, ssrc, s0, scale_dma, my_slot, my_scales);

    // int8: lo[m][l] are the 8 lanes.  int4: lo/hi are the two 8-lane halves.
    float lo[MT][8], hi[MT][8], gacc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        gacc[m] = 0.0f;
#pragma unroll
        for (int l = 0; l < 8; ++l) lo[m][l] = hi[m][l] = 0.0f;
    }
    const size_t K = (size_t)p.K;
    const uint32_t magic = opaque_magic();

    for (int s = s0; s < s1; ++s) {
        wait_vmcnt<0>();   // stripe s (and its scales) landed in the slot
        u32x4 mine[kLoads];
#pragma unroll
        for (int j = 0; j < kLoads; ++j) mine[j] = my_slot[8 * lane + (j ^ swz)];
        float gscale[F::scale_words];
        if constexpr (F::group) {
            if (scale_dma) {
                if constexpr (FMT == F_W4G128) {
                    gscale[0] = my_scales[lane];
                    gscale[1] = my_scales[64 + lane];
                } else {
                    const f32x4 v0 = ((const f32x4 *)my_scales)[lane];
                    const f32x4 v1 = ((const f32x4 *)(my_scales + 256))[lane];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        gscale[e] = v0[e];
                        gscale[4 + e] = v1[e];
                    }
                }
            }
        }
        // The slot is refilled only once every lane's reads have returned.
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
        if (s + 1 < s1) issue_stripe<FMT>(src, ssrc, s + 1, scale_dma, my_slot, my_scales);

        if constexpr (F::w8) {
            // 128 int8 weights: k = 128s + 4d + j belongs to lane 4(d&1) + j.
            const size_t kb = (size_t)s * kStripe;
#pragma unroll
            for (int d = 0; d < 32; ++d) {
                const uint32_t x = mine[d >> 2][d & 3];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float w = (float)(int)(int8_t)(uint8_t)(x >> (8 * j));
                    const int l = 4 * (d & 1) + j;
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        const size_t k = (size_t)(m0 + m) * K + kb + 4 * d + j;
                        float a;
                        if constexpr (FMT == F_W8A32) {
                            a = ((const cf32 *)as_const(p.A))[k];
                        } else {
                            const uint32_t pr = as_const(p.A)[k >> 1];
                            a = (j & 1) ? bf16_hi(pr) : bf16_lo(pr);
                        }
                        lo[m][l] = __builtin_fmaf(a, w, lo[m][l]);
                    }
                }
            }
        } else {
            // Activations arrive in batches of kBatch chunks per row (one
            // round of scalar loads per batch, immediate offsets from a
            // per-stripe base).
            constexpr int kBatch = (MT == 1) ? 8 : (MT == 2 ? 4 : 2);
            constexpr int kChunksPerGroup = (FMT == F_W4G32) ? 2 : 8;
            const size_t row_dw = K / 2;                                     // dwords per activation row
            const cu32 *ab = as_const(p.A) + (size_t)m0 * row_dw + (size_t)s * kStripe;
#pragma unroll
            for (int cb = 0; cb < 16; cb += kBatch) {
                uint32_t act[MT][8 * kBatch];
#pragma unroll
                for (int m = 0; m < MT; ++m)
#pragma unroll
                    for (int j = 0; j < 8 * kBatch; ++j) act[m][j] = ab[m * row_dw + 8 * cb + j];
#pragma unroll
                for (int c = cb; c < cb + kBatch; ++c) {
                    w4_chunk<MT, 8 * kBatch>(mine[c >> 1][2 * (c & 1)], mine[c >> 1][2 * (c & 1) + 1],
                                             &act[0][8 * (c - cb)], magic, lo, hi);
                    if constexpr (F::group) {
                        if ((c + 1) % kChunksPerGroup == 0) {
                            const int gl = c / kChunksPerGroup;                 // group within the stripe
                            const int g = F::groups_per_stripe * s + gl;
                            if (!global_split) {
                                if (wave == 0) {
#pragma unroll
                                    for (int m = 0; m < MT; ++m)
                                        gacc[m] =
                                            __builtin_fmaf(w4_block_and_reset(lo[m], hi[m]), gscale[gl], gacc[m]);
                                } else {
                                    // a later part of a locally split tile: park the block sums
                                    const int gi = g - G0;
#pragma unroll
                                    for (int m = 0; m < MT; ++m)
                                        fold_blocks[(gi * MT + m) * 64 + lane] = w4_block_and_reset(lo[m], hi[m]);
                                    fold_scales[gi * 64 + lane] = gscale[gl];
                                }
                            } else {
#pragma unroll
                                for (int m = 0; m < MT; ++m) {
                                    const float block = w4_block_and_reset(lo[m], hi[m]);
                                    if (n < p.N)
                                        __hip_atomic_store(p.P + ((size_t)g * p.M + m0 + m) * p.N + n, block,
                                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                                }
                            }
                        }
                    }
                }
            }
        }
    }

    if constexpr (F::group) {
        if (local_split) {
            // Every part of the tile has parked its block sums; part 0 folds
            // them after its own groups, in group order.
            __syncthreads();
            if (wave != 0) return;
            for (int gi = 0; gi < p.G - G0; ++gi) {
                const float sc = fold_scales[gi * 64 + lane];
#pragma unroll
                for (int m = 0; m < MT; ++m) gacc[m] = __builtin_fmaf(fold_blocks[(gi * MT + m) * 64 + lane], sc, gacc[m]);
            }
        } else if (global_split) {
            // The block sums went out as agent-scope stores (written through
            // to the device-coherent level, no L2 write-back needed); once
            // they have completed (vmcnt 0) the wave takes a ticket.  The last
            // of the tile's parts reads every block back with agent-scope
            // loads and folds the groups in order.
            wait_vmcnt<0>();
            int ticket = 0;
            if (lane == 0)
                ticket = __hip_atomic_fetch_add(p.T + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ticket = __builtin_amdgcn_readfirstlane(ticket);
            if (ticket != nparts - 1) return;
            if (n < p.N) {
                const size_t gstride = (size_t)p.M * p.N;
                const float *srow = p.S + (size_t)n * p.G;
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    float *pp = p.P + (size_t)(m0 + m) * p.N + n;
                    float acc = 0.0f;
#pragma unroll 8
                    for (int g = 0; g < p.G; ++g)
                        acc = __builtin_fmaf(
                            __hip_atomic_load(pp + g * gstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), srow[g],
                            acc);
                    ((uint16_t *)p.C)[(size_t)(m0 + m) * p.N + n] = f32_to_bf16(acc);
                }
            }
            if (lane == 0) __hip_atomic_store(p.T + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
    }

    if (n >= p.N) return;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const size_t o = (size_t)(m0 + m) * p.N + n;
        if constexpr (FMT == F_W8A32) {
            ((float *)p.C)[o] = hsum8(lo[m]) * p.S[n];
        } else if constexpr (FMT == F_W8A16) {
            ((uint16_t *)p.C)[o] = f32_to_bf16(hsum8(lo[m]) * p.S[n]);
        } else if constexpr (FMT == F_W4ROW) {
            ((uint16_t *)p.C)[o] = f32_to_bf16(w4_block_and_reset(lo[m], hi[m]) * p.S[n]);
        } else {
            ((uint16_t *)p.C)[o] = f32_to_bf16(gacc[m]);
        }
    }
}

constexpr size_t kMaxLds = 160 * 1024;   // LDS per workgroup on gfx950

// ----------------------------------------------------- small-M group GEMM
// For a few activation rows (MTP verify, short prefills: M >= 3 below the
// matrix-core threshold) the group formats are bound by the FMAs, M per
// weight, not by the weight stream.  Lane = row as above, but the
// activations reach the lanes through DPP instead of scalar loads: lane i of
// every 16-lane row of the wave holds element i of the current 16-element
// chunk of activation row m, and v_fmac_f32_dpp row_newbcast:l hands element l
// to all 64 lanes inside the FMA itself (one instruction per product, the same
// single rounding as fmaf).  The chunk's 16 weights are decoded once per lane
// and used by the wave's MT activation rows, whose bf16 values for the
// stripe arrive by DMA beside the weights, double-buffered in LDS.  The first
// chunk of a group multiplies instead of adding to zero: fma(a, w, +0) and
// a * w differ only in the sign of a zero, and a zero block sum of either
// sign leaves the group fold fma(block, scale, acc) unchanged (acc starts at
// +0), so the outputs keep every bit.  The m-groups of MT rows are the grid's
// second dimension (their weight reads meet in the caches); K is divided
// among the waves of a workgroup as in the exact kernel, parts 1.. park
// their block sums in LDS and part 0 folds them in group order.

// Eight products of one chunk half: acc[l] (op)= a of lane B + l of this
// 16-lane row times w[l].  The s_nop covers the two wait states a DPP source
// needs after a VALU write.
#define PILM_BC8(OP, B0, B1, B2, B3, B4, B5, B6, B7, CONS)                                                         \
    asm volatile("s_nop 1\n\t"                                                                                    \
                 OP " %0, %8, %9 row_newbcast:" #B0 " row_mask:0xf bank_mask:0xf\n\t"                             \
                 OP " %1, %8, %10 row_newbcast:" #B1 " row_mask:0xf bank_mask:0xf\n\t"                            \
                 OP " %2, %8, %11 row_newbcast:" #B2 " row_mask:0xf bank_mask:0xf\n\t"                            \
                 OP " %3, %8, %12 row_newbcast:" #B3 " row_mask:0xf bank_mask:0xf\n\t"                            \
                 OP " %4, %8, %13 row_newbcast:" #B4 " row_mask:0xf bank_mask:0xf\n\t"                            \
                 OP " %5, %8, %14 row_newbcast:" #B5 " row_mask:0xf bank_mask:0xf\n\t"                            \
                 OP " %6, %8, %15 row_newbcast:" #B6 " row_mask:0xf bank_mask:0xf\n\t"                            \
                 OP " %7, %8, %16 row_newbcast:" #B7 " row_mask:0xf bank_mask:0xf"                                \
                 : CONS(acc[0]), CONS(acc[1]), CONS(acc[2]), CONS(acc[3]), CONS(acc[4]), CONS(acc[5]),           \
                   CONS(acc[6]), CONS(acc[7])                                                                     \
                 : "v"(a), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]))
#define PILM_RW(x) "+v"(x)
#define PILM_WO(x) "=&v"(x)

template <int B, bool FIRST>
__device__ __forceinline__ void bcast8(float (&acc)[8], float a, const float (&w)[8]) {
    if constexpr (B == 0 && FIRST)
        PILM_BC8("v_mul_f32_dpp", 0, 1, 2, 3, 4, 5, 6, 7, PILM_WO);
    else if constexpr (B == 0)
        PILM_BC8("v_fmac_f32_dpp", 0, 1, 2, 3, 4, 5, 6, 7, PILM_RW);
    else if constexpr (FIRST)
        PILM_BC8("v_mul_f32_dpp", 8, 9, 10, 11, 12, 13, 14, 15, PILM_WO);
    else
        PILM_BC8("v_fmac_f32_dpp", 8, 9, 10, 11, 12, 13, 14, 15, PILM_RW);
}
#undef PILM_BC8
#undef PILM_RW
#undef PILM_WO

__device__ __forceinline__ float w4_block(const float (&lo)[8], const float (&hi)[8]) {
    float s[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) s[l] = lo[l] + hi[l];
    return hsum8(s);
}

// bf16 bytes of one stripe of MT activation rows, and of its two buffers.
template <int MT>
constexpr int bcast_act_bytes() { return 2 * MT * 256 * 2; }

// LDS: pl stripe slots, pl activation buffers, then (pl > 1) the fold area:
// float blocks[G - G0][MT][64] and float scales[G - G0][64], G0 = groups of
// part 0.
// WIN (windowed fold, for long rows whose parked block sums would not fit):
// the waves take stripes in rounds, wave w stripe t * pl + w of round t, and
// park each round's block sums in one of two buffers,
// float blocks[2][pl][GPS][MT][64] and scales[2][pl][GPS][64]; after the
// round's barrier wave 0 folds them in stripe and group order while the
// others go on to the next round in the other buffer (a buffer is written
// again only after the next barrier, which wave 0 reaches after its fold).
template <int FMT, int MT, bool WIN = false>
__global__ __launch_bounds__(64 * kMaxParts) void gemv_bcast_kernel(const uint16_t *__restrict__ A,
                                                                   const uint8_t *__restrict__ W,
                                                                   const float *__restrict__ S,
                                                                   uint16_t *__restrict__ C, int M, int N, int K,
                                                                   int sps) {
    using F = StripeFmt<FMT>;
    constexpr int GPS = F::groups_per_stripe;   // 2 (g128) or 8 (g32)
    constexpr int CPG = 16 / GPS;               // 16-element chunks per group
    constexpr int kAct = bcast_act_bytes<MT>();
    constexpr int kActLoads = MT / 2;           // 1 KB DMA instructions per stripe: two rows each
    extern __shared__ __align__(16) unsigned char lds[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int pl = (int)(blockDim.x >> 6);
    const int row0 = blockIdx.x * 64;
    const int n = row0 + lane;
    const int nc = n < N ? n : N - 1;
    const int mb = (int)blockIdx.y * MT;        // first activation row of this workgroup
    const int mvalid = min(MT, M - mb);
    const int nstripes = K / 256;
    const int G = nstripes * GPS;
    const int s0 = WIN ? min(wave, nstripes) : min(wave * sps, nstripes);
    const int s1 = WIN ? nstripes : min(s0 + sps, nstripes);
    const int sstep = WIN ? pl : 1;                 // a wave's next stripe
    const int nrounds = (nstripes + pl - 1) / pl;   // (WIN)
    const int G0 = min(sps * GPS, G);
    const size_t row_bytes = (size_t)K / 2;

    const uint8_t *src[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int r = 8 * i + (lane >> 3);
        const int q = (lane & 7) ^ ((r >> 1) & 7);
        src[i] = W + (size_t)min(row0 + r, N - 1) * row_bytes + q * 16;
    }
    const int swz = (lane >> 1) & 7;
    u32x4 *my_slot = (u32x4 *)(lds + wave * kSlotBytes);
    unsigned char *my_act = lds + pl * kSlotBytes + wave * kAct;   // [2][MT rows][256] bf16
    float *fold_blocks = (float *)(lds + pl * (kSlotBytes + kAct));
    float *fold_scales = fold_blocks + (WIN ? (size_t)2 * pl * GPS * MT * 64 : (size_t)(G - G0) * MT * 64);
    const float *srow = S + (size_t)nc * G;
    // Activation DMA: instruction j, lane t fetches 16 bytes of row 2j + t/32
    // (rows past M repeat the last row; their results are not stored).
    const uint16_t *asrc[kActLoads];
#pragma unroll
    for (int j = 0; j < kActLoads; ++j)
        asrc[j] = A + (size_t)(mb + min(2 * j + (lane >> 5), mvalid - 1)) * K + 8 * (lane & 31);

    auto issue = [&](int st) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(src[i] + (size_t)st * kStripe),
                                             (lds_void *)(my_slot + 64 * i), 16, 0, kNT);
#pragma unroll
        for (int j = 0; j < kActLoads; ++j)
            __builtin_amdgcn_global_load_lds((const void *)(asrc[j] + (size_t)st * 256),
                                             (lds_void *)(my_act + (((st - s0) / sstep) & 1) * (kAct / 2) + j * 1024), 16, 0,
                                             0);
    };
    if (s0 < s1) issue(s0);

    float lo[MT][8], hi[MT][8], gacc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) gacc[m] = 0.0f;
    const uint32_t magic = opaque_magic();

    auto fold_round = [&](int t) {   // (WIN) wave 0: round t's block sums, stripe then group order
        const float *pb = fold_blocks + (size_t)(t & 1) * pl * GPS * MT * 64;
        const float *ps = fold_scales + (size_t)(t & 1) * pl * GPS * 64;
        for (int w = 0; w < pl && t * pl + w < nstripes; ++w)
#pragma unroll
            for (int gl = 0; gl < GPS; ++gl) {
                const float scg = ps[(w * GPS + gl) * 64 + lane];
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    gacc[m] = __builtin_fmaf(pb[((w * GPS + gl) * MT + m) * 64 + lane], scg, gacc[m]);
            }
    };
#pragma unroll 1
    for (int it = 0, s = s0; WIN ? it < nrounds : s < s1; ++it, s += sstep) {
        if (WIN && s >= s1) {   // no stripe for this wave in the last round
            __syncthreads();
            if (wave == 0) fold_round(it);
            continue;
        }
        float sc[GPS];
#pragma unroll
        for (int g = 0; g < GPS; ++g) sc[g] = srow[s * GPS + g];
        wait_vmcnt<0>();   // stripe s and its activations landed (and the scales arrived)
        u32x4 mine[kLoads];
#pragma unroll
        for (int j = 0; j < kLoads; ++j) mine[j] = my_slot[8 * lane + (j ^ swz)];
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the slot may be refilled
        if (s + sstep < s1) issue(s + sstep);

        // lane i of each 16-lane row reads element i of every chunk
        const uint16_t *abuf = (const uint16_t *)(my_act + (it & 1) * (kAct / 2)) + (lane & 15);
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            float a[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) a[m] = __uint_as_float((uint32_t)abuf[m * 256 + 16 * c] << 16);
            h2 ql[4], qh[4];
            dequant_w4(mine[c >> 1][2 * (c & 1)], magic, ql);
            dequant_w4(mine[c >> 1][2 * (c & 1) + 1], magic, qh);
            float wl[8], wh[8];
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                wl[l] = (float)ql[l].x;
                wl[l + 4] = (float)ql[l].y;
                wh[l] = (float)qh[l].x;
                wh[l + 4] = (float)qh[l].y;
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                if (c % CPG == 0) {
                    bcast8<0, true>(lo[m], a[m], wl);
                    bcast8<8, true>(hi[m], a[m], wh);
                } else {
                    bcast8<0, false>(lo[m], a[m], wl);
                    bcast8<8, false>(hi[m], a[m], wh);
                }
            }
            if ((c + 1) % CPG == 0) {
                const int gl = c / CPG;
                const int g = GPS * s + gl;
                if constexpr (WIN) {
                    float *pb = fold_blocks + (size_t)(it & 1) * pl * GPS * MT * 64;
#pragma unroll
                    for (int m = 0; m < MT; ++m) pb[((wave * GPS + gl) * MT + m) * 64 + lane] = w4_block(lo[m], hi[m]);
                    fold_scales[((size_t)(it & 1) * pl * GPS + wave * GPS + gl) * 64 + lane] = sc[gl];
                } else {
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        const float block = w4_block(lo[m], hi[m]);
                        if (wave == 0)
                            gacc[m] = __builtin_fmaf(block, sc[gl], gacc[m]);
                        else
                            fold_blocks[((g - G0) * MT + m) * 64 + lane] = block;
                    }
                    if (wave != 0) fold_scales[(g - G0) * 64 + lane] = sc[gl];
                }
            }
        }
        if constexpr (WIN) {
            __syncthreads();
            if (wave == 0) fold_round(it);
        }
    }

    if (WIN) {
        if (wave != 0) return;
    } else if (pl > 1) {
        __syncthreads();
        if (wave != 0) return;
        for (int gi = 0; gi < G - G0; ++gi) {
            const float scg = fold_scales[gi * 64 + lane];
#pragma unroll
            for (int m = 0; m < MT; ++m) gacc[m] = __builtin_fmaf(fold_blocks[(gi * MT + m) * 64 + lane], scg, gacc[m]);
        }
    }
    if (n >= N) return;
#pragma unroll
    for (int m = 0; m < MT; ++m)
        if (m < mvalid) C[(size_t)(mb + m) * N + n] = f32_to_bf16(gacc[m]);
}

static size_t bcast_lds_bytes(int mt, int pl, int sps, int G, int gps) {
    size_t bytes = (size_t)pl * (kSlotBytes + (size_t)2 * mt * 256 * 2);
    if (pl > 1) bytes += (size_t)(G - std::min(sps * gps, G)) * 64 * (mt + 1) * sizeof(float);
    return bytes;
}

// Windowed fold: two round buffers of pl stripes' block sums and scales.
static size_t bcast_win_lds_bytes(int mt, int pl, int gps) {
    return (size_t)pl * (kSlotBytes + (size_t)2 * mt * 256 * 2) + (size_t)2 * pl * gps * 64 * (mt + 1) * sizeof(float);
}

template <int FMT, int MT, bool WIN>
static int launch_bcast_one(dim3 grid, dim3 block, size_t lds, hipStream_t st, const uint16_t *A, const uint8_t *W,
                            const float *S, uint16_t *C, int M, int N, int K, int sps) {
    static std::once_flag once;
    static hipError_t attr_rc = hipSuccess;
    std::call_once(once, [] {
        attr_rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_bcast_kernel<FMT, MT, WIN>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
    });
    if (attr_rc != hipSuccess) return ECPU_ERR_DEVICE;
    gemv_bcast_kernel<FMT, MT, WIN><<<grid, block, lds, st>>>(A, W, S, C, M, N, K, sps);
    return ECPU_OK;
}

template <int FMT, int MT>
static int launch_bcast(bool win, dim3 grid, dim3 block, size_t lds, hipStream_t st, const uint16_t *A,
                        const uint8_t *W, const float *S, uint16_t *C, int M, int N, int K, int sps) {
    return win ? launch_bcast_one<FMT, MT, true>(grid, block, lds, st, A, W, S, C, M, N, K, sps)
               : launch_bcast_one<FMT, MT, false>(grid, block, lds, st, A, W, S, C, M, N, K, sps);
}

// Small-M path of the group formats: every M rows in one launch (m-groups of
// MT = 4 or 8 rows on the grid's y dimension), K divided among up to 8 waves
// per tile (fewer when the parked block sums would not fit LDS).  A wave's
// work grows with MT, so the eight-row waves are taken only where there are
// enough of them to fill the SIMDs (>= 1536 waves) and add no padding rows
// over MT = 4 (measured at M = 16:
// 6144x2048 16.4 vs 21.0 us, 4096x2048 16.3 vs 11.2 us).  The group-quad
// kernels take (returns ECPU_ERR_UNSUPPORTED): up to four rows with fewer
// than 768 waves or at most 6144 rows (g128 4096x4096 M=4: 13.0 vs 16.1 us,
// 6144x2048 M=3: 9.8 vs 11.0 us), up to eight rows when LDS leaves two waves
// per tile or fewer and the windowed fold is not available (or takes any
// beyond 8192 rows: those go to the 64-row tiles, g32 12288x2048 M=5 22.6 vs
// 29.8 us), and five rows on small cramped shapes (below).
static int run_bcast(int fmt, size_t M, size_t N, size_t K, const void *A, const uint8_t *W, const float *S, void *C,
                     hipStream_t st, const char *fn) {
    const int nstripes = (int)(K / 256);
    const int gps = fmt == F_W4G128 ? 2 : 8;
    const int G = nstripes * gps;
    const size_t ntiles = (N + 63) / 64;
    bool reduced = false;   // LDS took waves from the four-row plan
    auto plan = [&](int mt, int &pl, int &sps) {
        pl = std::min(kMaxParts, nstripes);
        const int env_pl = env_int("PILM_HIP_BCAST_PL", 0);
        if (env_pl >= 1 && env_pl <= kMaxParts) pl = std::min(env_pl, nstripes);
        sps = (nstripes + pl - 1) / pl;
        pl = (nstripes + sps - 1) / sps;   // every part gets a stripe
        while (pl > 1 && bcast_lds_bytes(mt, pl, sps, G, gps) > kMaxLds) {
            pl = (pl + 1) / 2;
            sps = (nstripes + pl - 1) / pl;
            pl = (nstripes + sps - 1) / sps;
            if (mt == 4) reduced = true;
        }
    };
    int pl8, sps8, pl4, sps4;
    plan(8, pl8, sps8);
    plan(4, pl4, sps4);
    // The windowed fold keeps more waves where the parked block sums would
    // not fit (group 32, long rows): the most parts (8, 4, 2) whose round
    // buffers fit, used for four-row groups when that beats the parked plan
    // (g32 4096x12288 M=16: 77 vs 266 us, 1024x4096 M=16: 27 vs 50 us; g128
    // 4096x12288 M=16: 51 vs 58 us).  Eight-row groups keep the parked plan:
    // their windowed buffers leave 2 waves and one workgroup per CU (g32
    // 24576x4096 M=32: 453 vs 239 us).
    auto win_parts = [&](int mt) {
        int p = std::min(kMaxParts, nstripes);
        while (p > 1 && bcast_win_lds_bytes(mt, p, gps) > kMaxLds) p /= 2;
        return p;
    };
    const int env_win = env_int("PILM_HIP_BCAST_WIN", -1);
    const int pl4_parked = pl4;
    const int pw8 = win_parts(8), pw4 = win_parts(4);
    const bool win8 = env_win == 1 && pw8 > 1;
    const bool win4 = env_win == 1 ? pw4 > 1 : (env_win != 0 && pw4 > pl4);
    if (win8) { pl8 = pw8; sps8 = (nstripes + pw8 - 1) / pw8; }
    if (win4) { pl4 = pw4; sps4 = (nstripes + pw4 - 1) / pw4; }
    const bool cramped = reduced && !win4 && (pl4 <= 2 || N > 8192);
    // five rows on a small shape whose parked plan keeps two waves or fewer:
    // two group-quad launches (4 + 1 rows) win (g32 1024x4096: 22.1 vs 26.7
    // us, 2048x6144: 32.6 vs 39.4 us)
    const bool five_gq = reduced && pl4_parked <= 2 && env_win != 1 && M == 5 && N <= 6144 && K <= 8192;
    // up to four rows stay here (windowed) when the 8-row group-quad kernel
    // could not take them in one launch (its LDS: rings, the rows, 8 rows'
    // scales and block sums; g32 4096x12288 M=4: 3 + 1 rows, 86 us)
    const bool gq8_one = (size_t)32768 + M * K * 2 + (size_t)8 * G * 4 * (1 + M) <= kMaxLds;
    const bool keep_small = win4 && !gq8_one;
    const size_t waves8 = ntiles * pl8 * ((M + 7) / 8), waves4 = ntiles * pl4 * ((M + 3) / 4);
    const size_t pad8 = (M + 7) / 8 * 8, pad4 = (M + 3) / 4 * 4;   // rows computed, padding included
    int mt = (pad8 <= pad4 && waves8 >= 1536) ? 8 : 4;
    const int env_mt = env_int("PILM_HIP_BCAST_MT", 0);
    if (env_mt == 4 || env_mt == 8)
        mt = env_mt;
    else if ((M <= 4 && (waves4 < 768 || N <= 6144) && !keep_small) || (M <= 8 && cramped) || five_gq)
        return ECPU_ERR_UNSUPPORTED;
    const int pl = mt == 8 ? pl8 : pl4, sps = mt == 8 ? sps8 : sps4;
    const bool win = mt == 8 ? win8 : win4;
    const size_t lds = win ? bcast_win_lds_bytes(mt, pl, gps) : bcast_lds_bytes(mt, pl, sps, G, gps);
    if (lds > kMaxLds) return fail(ECPU_ERR_DEVICE, "%s: small-M tile does not fit in LDS", fn);
    const size_t mgroups = (M + mt - 1) / mt;
    if (mgroups > 65535) return ECPU_ERR_UNSUPPORTED;
    const dim3 grid((unsigned)((N + 63) / 64), (unsigned)mgroups);
    const dim3 block((unsigned)(64 * pl));
    const uint16_t *a16 = (const uint16_t *)A;
    uint16_t *c16 = (uint16_t *)C;
    int rc;
    if (fmt == F_W4G128)
        rc = mt == 4 ? launch_bcast<F_W4G128, 4>(win, grid, block, lds, st, a16, W, S, c16, (int)M, (int)N, (int)K, sps)
                     : launch_bcast<F_W4G128, 8>(win, grid, block, lds, st, a16, W, S, c16, (int)M, (int)N, (int)K, sps);
    else
        rc = mt == 4 ? launch_bcast<F_W4G32, 4>(win, grid, block, lds, st, a16, W, S, c16, (int)M, (int)N, (int)K, sps)
                     : launch_bcast<F_W4G32, 8>(win, grid, block, lds, st, a16, W, S, c16, (int)M, (int)N, (int)K, sps);
    if (rc != ECPU_OK) return fail(ECPU_ERR_DEVICE, "%s: raising the LDS limit of the small-M kernel failed", fn);
    return ECPU_OK;
}

// ----------------------------------------------------- literal fallback
__device__ __forceinline__ float nib(const uint8_t *w, size_t k) {
    const uint8_t b = w[k >> 1];
    const int v = (k & 1) ? (b >> 4) : (b & 0x0F);
    return (float)(v >= 8 ? v - 16 : v);
}

__device__ __forceinline__ float bf16_at(const uint16_t *a, size_t k) { return __uint_as_float((uint32_t)a[k] << 16); }

__device__ float dot_i4_literal(const uint16_t *a, const uint8_t *w, size_t K) {
    float lo[8] = {0, 0, 0, 0, 0, 0, 0, 0}, hi[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t k = 0;
    for (; k + 16 <= K; k += 16) {
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            lo[l] = __builtin_fmaf(bf16_at(a, k + l), nib(w, k + l), lo[l]);
            hi[l] = __builtin_fmaf(bf16_at(a, k + 8 + l), nib(w, k + 8 + l), hi[l]);
        }
    }
    float s[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) s[l] = lo[l] + hi[l];
    float out = hsum8(s);
    for (; k + 1 < K; k += 2) {
        out = __builtin_fmaf(bf16_at(a, k), nib(w, k), out);
        out = __builtin_fmaf(bf16_at(a, k + 1), nib(w, k + 1), out);
    }
    if (k < K) out = __builtin_fmaf(bf16_at(a, k), nib(w, k), out);
    return out;
}

template <int FMT>
__global__ __launch_bounds__(256) void gemv_literal_kernel(GemvArgs p, int group_size) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)p.M * p.N) return;
    const size_t m = idx / p.N, n = idx % p.N;
    const size_t K = (size_t)p.K;
    if constexpr (FMT == F_W8A32 || FMT == F_W8A16) {
        const int8_t *w = (const int8_t *)p.W + n * K;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        size_t k = 0;
        for (; k + 8 <= K; k += 8) {
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                const float a = (FMT == F_W8A32) ? ((const float *)p.A)[m * K + k + l]
                                                 : bf16_at((const uint16_t *)p.A, m * K + k + l);
                acc[l] = __builtin_fmaf(a, (float)w[k + l], acc[l]);
            }
        }
        float out = hsum8(acc);
        for (; k < K; ++k) {
            const float a = (FMT == F_W8A32) ? ((const float *)p.A)[m * K + k]
                                             : bf16_at((const uint16_t *)p.A, m * K + k);
            out = __builtin_fmaf(a, (float)w[k], out);
        }
        if constexpr (FMT == F_W8A32)
            ((float *)p.C)[idx] = out * p.S[n];
        else
            ((uint16_t *)p.C)[idx] = f32_to_bf16(out * p.S[n]);
    } else {
        const uint16_t *a = (const uint16_t *)p.A + m * K;
        const uint8_t *w = p.W + n * (size_t)p.row_bytes;
        if constexpr (FMT == F_W4ROW) {
            ((uint16_t *)p.C)[idx] = f32_to_bf16(dot_i4_literal(a, w, K) * p.S[n]);
        } else {
            const size_t G = (K + group_size - 1) / group_size;
            float acc = 0.0f;
            for (size_t g = 0; g < G; ++g) {
                const size_t k0 = g * group_size;
                const size_t gk = K - k0 < (size_t)group_size ? K - k0 : (size_t)group_size;
                acc = __builtin_fmaf(dot_i4_literal(a + k0, w + k0 / 2, gk), p.S[n * G + g], acc);
            }
            ((uint16_t *)p.C)[idx] = f32_to_bf16(acc);
        }
    }
}

// --------------------------------------------------------------- launch


template <int FMT, int MT>
static int launch_one(dim3 grid, dim3 block, size_t lds, hipStream_t st, const GemvArgs &a, int m0) {
    // Dynamic LDS above the default limit has to be allowed once per kernel.
    static std::once_flag once;
    static hipError_t attr_rc = hipSuccess;
    std::call_once(once, [] {
        attr_rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_exact_kernel<FMT, MT>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
    });
    if (attr_rc != hipSuccess) return ECPU_ERR_DEVICE;
    gemv_exact_kernel<FMT, MT><<<grid, block, lds, st>>>(a.A, a.W, a.S, a.C, a.P, a.T, a, m0);
    return ECPU_OK;
}

template <int FMT>
static int launch_exact_mt(int mt, dim3 grid, dim3 block, size_t lds, hipStream_t st, const GemvArgs &a, int m0) {
    switch (mt) {
        case 1: return launch_one<FMT, 1>(grid, block, lds, st, a, m0);
        case 2: return launch_one<FMT, 2>(grid, block, lds, st, a, m0);
        case 3: return launch_one<FMT, 3>(grid, block, lds, st, a, m0);
        default: return launch_one<FMT, 4>(grid, block, lds, st, a, m0);
    }
}

static int launch_exact(int fmt, int mt, dim3 grid, dim3 block, size_t lds, hipStream_t st, const GemvArgs &a,
                        int m0) {
    switch (fmt) {
        case F_W8A32: return launch_exact_mt<F_W8A32>(mt, grid, block, lds, st, a, m0);
        case F_W8A16: return launch_exact_mt<F_W8A16>(mt, grid, block, lds, st, a, m0);
        case F_W4ROW: return launch_exact_mt<F_W4ROW>(mt, grid, block, lds, st, a, m0);
        case F_W4G128: return launch_exact_mt<F_W4G128>(mt, grid, block, lds, st, a, m0);
        default: return launch_exact_mt<F_W4G32>(mt, grid, block, lds, st, a, m0);
    }
}

// Dynamic LDS of one workgroup: stripe slots and scale slots of its pl waves,
// plus the fold area when a tile is split inside the workgroup.
static size_t exact_lds_bytes(const GemvArgs &a, int groups_per_stripe, int mt) {
    size_t bytes = (size_t)a.pl * (kSlotBytes + a.scale_slot_bytes);
    if (a.pg == 1 && a.pl > 1) {
        const int g0 = std::min(a.sps * groups_per_stripe, a.G);
        bytes += (size_t)(a.G - g0) * 64 * (mt + 1) * sizeof(float);
    }
    return bytes;
}

// ---- per-call timing (HIP events on the launch stream) -------------------
// Enabled by ecpu_hip_profile_begin(); each linear call records one event
// pair around its kernels, tagged with a family name and the call's
// algorithmic bytes and flops.  Read back with ecpu_hip_profile_read().
struct ProfRec {
    hipEvent_t a, b;
    const char *family;
    double bytes, flops;
};
static std::mutex g_prof_mu;
static std::vector<ProfRec> g_prof;
static std::vector<hipEvent_t> g_event_pool;
static bool g_prof_on = false;

static hipEvent_t pooled_event() {
    if (!g_event_pool.empty()) {
        hipEvent_t e = g_event_pool.back();
        g_event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    (void)hipEventCreate(&e);
    return e;
}

static const char *mfma_family_name(int fmt) {
    static const char *names[5] = {"w8a32_mfma", "w8a16_mfma", "w4a16_mfma", "w4a16g128_mfma", "w4a16g32_mfma"};
    return names[fmt];
}

static const char *family_name(int fmt, size_t M) {
    static const char *names[5][3] = {
        {"w8a32_gemv", "w8a32_m2to4", "w8a32_m5plus"},
        {"w8a16_gemv", "w8a16_m2to4", "w8a16_m5plus"},
        {"w4a16_gemv", "w4a16_m2to4", "w4a16_m5plus"},
        {"w4a16g128_gemv", "w4a16g128_m2to4", "w4a16g128_m5plus"},
        {"w4a16g32_gemv", "w4a16g32_m2to4", "w4a16g32_m5plus"}};
    return names[fmt][M == 1 ? 0 : (M <= 4 ? 1 : 2)];
}

hipEvent_t prof_begin(hipStream_t st) {
    if (!g_prof_on) return nullptr;
    std::lock_guard<std::mutex> lk(g_prof_mu);
    hipEvent_t ev0 = pooled_event();
    (void)hipEventRecord(ev0, st);
    return ev0;
}

void prof_end(hipEvent_t ev0, hipStream_t st, const char *family, double bytes, double flops) {
    if (!ev0) return;
    std::lock_guard<std::mutex> lk(g_prof_mu);
    if (!family) {   // nothing to file: the start event goes back to the pool
        g_event_pool.push_back(ev0);
        return;
    }
    hipEvent_t ev1 = pooled_event();
    (void)hipEventRecord(ev1, st);
    g_prof.push_back({ev0, ev1, family, bytes, flops});
}

int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return (v && *v) ? atoi(v) : dflt;
}

// Entry point shared by the five linear formats; arguments are validated by
// the caller (shapes, device residency, buffer extents).
int run_linear(int fmt, size_t M, size_t N, size_t K, const void *A, const uint8_t *W, const float *S,
               void *C, const char *fn) {
    if (M == 0 || N == 0) return ECPU_OK;
    hipStream_t st = current_stream();
    const bool w8 = (fmt == F_W8A32 || fmt == F_W8A16);
    const int group = (fmt == F_W4G128) ? 128 : (fmt == F_W4G32 ? 32 : 0);
    GemvArgs a;
    a.A = A;
    a.W = W;
    a.S = S;
    a.C = C;
    a.P = nullptr;
    a.T = nullptr;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.row_bytes = (int)(w8 ? K : (K + 1) / 2);
    a.G = group ? (int)((K + group - 1) / group) : 0;
    a.ntiles = (int)((N + 63) / 64);

    const size_t stripe_k = w8 ? kStripe : 2 * kStripe;   // weights per 128-byte stripe
    const bool aligned = (((uintptr_t)W | (uintptr_t)A) & 15) == 0 &&
                         (fmt != F_W4G32 || ((uintptr_t)S & 15) == 0) && ((uintptr_t)S & 3) == 0;
    const bool fast = K > 0 && K % stripe_k == 0 && aligned && env_int("PILM_HIP_LITERAL", 0) == 0;
    // Prefill / verify shapes go to the matrix cores (within 1e-2 of the
    // reference); decode shapes stay on the exact kernels.
    const int min_m = mfma_min_m();
    const bool use_mfma = min_m > 0 && M >= (size_t)min_m && mfma_supports(K, A, W) &&
                          env_int("PILM_HIP_LITERAL", 0) == 0;
    if (!fast && !use_mfma) {
        const size_t total = M * N;
        switch (fmt) {
            case F_W8A32: gemv_literal_kernel<F_W8A32><<<(total + 255) / 256, 256, 0, st>>>(a, 0); break;
            case F_W8A16: gemv_literal_kernel<F_W8A16><<<(total + 255) / 256, 256, 0, st>>>(a, 0); break;
            case F_W4ROW: gemv_literal_kernel<F_W4ROW><<<(total + 255) / 256, 256, 0, st>>>(a, 0); break;
            case F_W4G128: gemv_literal_kernel<F_W4G128><<<(total + 255) / 256, 256, 0, st>>>(a, 128); break;
            default: gemv_literal_kernel<F_W4G32><<<(total + 255) / 256, 256, 0, st>>>(a, 32); break;
        }
        return check_launch(fn);
    }

    a.nstripes = (int)(K / stripe_k);
    a.pl = 1;
    a.pg = 1;
    a.sps = a.nstripes;
    a.scale_slot_bytes = fmt == F_W4G128 ? 2 * 64 * 4 : (fmt == F_W4G32 ? 8 * 64 * 4 : 0);
    const int groups_per_stripe = fmt == F_W4G128 ? 2 : (fmt == F_W4G32 ? 8 : 0);
    if (group && !use_mfma) {
        // K is divided among the waves of one workgroup (block sums meet in
        // LDS): 4 parts per tile once there are >= 256 tiles, which lets the
        // hardware balance quarter tiles across SIMDs, 8 below that.  Few
        // tiles with long rows are also divided across workgroups (block
        // sums meet in global memory), aiming at ~1024 waves, as long as every
        // part keeps a stripe.  (Chosen from measured per-shape times.)
        int pl = a.ntiles >= 256 ? 4 : kMaxParts;
        pl = std::min(pl, a.nstripes);
        const int spw = (a.nstripes + pl - 1) / pl;
        int pg = 1;
        if (a.ntiles < 256 && spw >= 3) pg = std::min(spw, (1024 + a.ntiles * pl - 1) / (a.ntiles * pl));
        const int env_pl = env_int("PILM_HIP_PL", 0), env_pg = env_int("PILM_HIP_PG", 0);
        const int env_ns = env_int("PILM_HIP_NSPLIT", 0);
        if (env_pl > 0 || env_pg > 0) {
            pl = std::max(1, std::min(env_pl > 0 ? env_pl : 1, kMaxParts));
            pg = std::max(1, env_pg > 0 ? env_pg : 1);
        } else if (env_ns > 0) {
            pl = 1;
            pg = env_ns;
        }
        pl = std::min(pl, a.nstripes);
        pg = std::max(1, std::min(pg, (a.nstripes + pl - 1) / pl));
        a.sps = (a.nstripes + pl * pg - 1) / (pl * pg);
        a.pl = pl;
        a.pg = pg;
        // A locally split tile parks the block sums of parts 1.. in LDS; fewer
        // parts when that would not fit (long K with group 32).
        while (a.pg == 1 && a.pl > 1 && exact_lds_bytes(a, groups_per_stripe, (int)std::min<size_t>(4, M)) > kMaxLds) {
            a.pl = (a.pl + 1) / 2;
            a.sps = (a.nstripes + a.pl - 1) / a.pl;
        }
    }
    if (a.pg > 1) {
        const int rc = split_scratch(st, (size_t)a.G * M * N, (size_t)a.ntiles, &a.P, &a.T, fn);
        if (rc != ECPU_OK) return rc;
    }
    const dim3 grid((unsigned)(a.ntiles * a.pg));
    const dim3 block((unsigned)(64 * a.pl));
    hipEvent_t ev0 = prof_begin(st);
    if (use_mfma) {
        const int rc = run_mfma(fmt, M, N, K, A, W, S, C, st, fn);
        if (rc != ECPU_OK) return rc;
    } else if (!group && env_int("PILM_HIP_ROWS", 1) != 0) {
        // per-row formats: the chains of a row are divided among four waves
        const int rc = run_rows(fmt, M, N, K, A, W, S, C, st, fn);
        if (rc != ECPU_OK) return rc;
    } else {
        // group formats up to 8192 rows: 16-row tiles, K divided among waves
        // (beyond that the 64-row tiles' cheaper decode wins, measured)
        int rc = ECPU_ERR_UNSUPPORTED;
        if (group && M >= 3 && env_int("PILM_HIP_BCAST", 1) != 0)
            rc = run_bcast(fmt, M, N, K, A, W, S, C, st, fn);
        // (two rows: the 64-row tiles from 6144 rows, 6144x2048 8.4 vs 10.0 us)
        if (rc == ECPU_ERR_UNSUPPORTED && group && env_int("PILM_HIP_GQ", N <= (M == 2 ? 4096u : 8192u) ? 1 : 0) != 0)
            rc = run_group_quad(fmt, M, N, K, A, W, S, C, st, fn);
        if (rc != ECPU_OK && rc != ECPU_ERR_UNSUPPORTED) return rc;
        if (rc == ECPU_ERR_UNSUPPORTED) {
            for (size_t m0 = 0; m0 < M; m0 += 4) {
                const int mt = (int)std::min<size_t>(4, M - m0);
                if (launch_exact(fmt, mt, grid, block, exact_lds_bytes(a, groups_per_stripe, mt), st, a, (int)m0) !=
                    ECPU_OK)
                    return fail(ECPU_ERR_DEVICE, "%s: raising the LDS limit of the GEMV kernel failed", fn);
            }
        }
    }
    if (ev0) {
        const double a_elt = (fmt == F_W8A32) ? 4.0 : 2.0;
        const double scale_bytes = 4.0 * (double)N * (group ? (double)a.G : 1.0);
        const double bytes = (double)N * a.row_bytes + scale_bytes + a_elt * (double)(M * K) + a_elt * (double)(M * N);
        prof_end(ev0, st, use_mfma ? mfma_family_name(fmt) : family_name(fmt, M), bytes,
                 2.0 * (double)M * (double)N * (double)K);
    }
    return check_launch(fn);
}

}  // namespace pilm

using namespace pilm;

extern "C" {

int ecpu_hip_profile_begin(void) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    for (auto &r : g_prof) {
        g_event_pool.push_back(r.a);
        g_event_pool.push_back(r.b);
    }
    g_prof.clear();
    g_prof_on = true;
    return ECPU_OK;
}

int ecpu_hip_profile_end(void) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    g_prof_on = false;
    return ECPU_OK;
}

// One line per family: "<family> <calls> <total_ms> <alg_bytes> <flops>".
int ecpu_hip_profile_read(char *buf, size_t len) {
    if (!buf || len == 0) return fail(ECPU_ERR_PARAM, "ecpu_hip_profile_read: empty buffer");
    std::lock_guard<std::mutex> lk(g_prof_mu);
    struct Agg {
        std::string name;
        long calls = 0;
        double ms = 0, bytes = 0, flops = 0;
    };
    std::vector<Agg> aggs;
    for (auto &r : g_prof) {
        if (hipEventSynchronize(r.b) != hipSuccess) return fail(ECPU_ERR_DEVICE, "profile: event sync failed");
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) return fail(ECPU_ERR_DEVICE, "profile: elapsed failed");
        Agg *g = nullptr;
        for (auto &x : aggs)
            if (x.name == r.family) g = &x;
        if (!g) {
            aggs.push_back(Agg{r.family});
            g = &aggs.back();
        }
        g->calls++;
        g->ms += ms;
        g->bytes += r.bytes;
        g->flops += r.flops;
    }
    std::string out;
    char line[256];
    for (auto &x : aggs) {
        snprintf(line, sizeof(line), "%s %ld %.6f %.0f %.0f\n", x.name.c_str(), x.calls, x.ms, x.bytes, x.flops);
        out += line;
    }
    if (out.size() + 1 > len) return fail(ECPU_ERR_PARAM, "ecpu_hip_profile_read: buffer too small");
    memcpy(buf, out.c_str(), out.size() + 1);
    return ECPU_OK;
}

}  // extern "C"
