// Exact GEMV / small-M GEMM for the per-row formats on gfx950: int8 weights
// with fp32 or bf16 activations (W8A32, W8A16) and nibble-packed int4 with
// one scale per row (W4A16, bundle v2).
//
// These formats accumulate every output row in independent FMA chains that
// each run over all of K -- 8 chains for int8 (chain l owns k = l mod 8,
// kernels.c:78-109, 330-393) and 16 for int4 (lo[l] owns k = 16c + l, hi[l]
// owns 16c + 8 + l, kernels.c:111-225) -- so K cannot be divided without
// changing the roundings.  The chains of a row are divided instead: a
// workgroup of four waves owns a tile of 64 rows (lane = row) and wave w owns
//   int8: chains 4(w>>1) + 2(w&1) + {0, 1}, i.e. bytes 2(w&1), 2(w&1)+1 of
//         the row's dwords of parity w>>1;
//   int4: the lo (w < 2) or hi (w >= 2) chains of every 16-element chunk,
//         nibble pairs (0,4),(1,5) for even w, (2,6),(3,7) for odd w.
// At the end the chains meet in LDS and wave 0 combines them exactly as the
// reference does: hsum ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)) of the 8 lanes
// (int4: of lo[l]+hi[l]), times the row scale, then bf16 for W8A16 / W4A16.
//
// The four waves stream the tile through a ring of D stripe slots (64 rows
// x 128 B each) filled by global -> LDS DMA; each wave issues two of a
// stripe's eight DMA instructions.  One barrier per stripe: once every wave
// has waited for its own part of stripe s, the stripe is complete in LDS, and
// every wave has finished reading stripe s-1, whose slot then receives
// stripe s+D-1.  D-1 stripes stay in flight per tile, enough to cover HBM
// latency when only a few tiles share the GPU.  Activations come through
// scalar loads (the same k for every lane), up to 32 dwords at a time.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <mutex>
#include <type_traits>

#include "cpu_order.h"
#include "gemv_device.h"
#include "internal.h"

namespace pilm {

namespace {

constexpr int kRowWaves = 4;                 // waves per tile, one per SIMD

template <int FMT, int MT>
struct RowPlan {
    static constexpr bool w8 = FMT != F_W4ROW;
    static constexpr int chains = w8 ? 2 : 4;                  // chains per wave
    static constexpr int apd = FMT == F_W8A16 ? 1 : 2;         // activation dwords per step and row
    static constexpr int sub = MT <= 1 ? 1 : (MT <= 2 ? 2 : 4);  // sub-blocks per stripe
    static constexpr int steps = 16 / sub;                     // row dwords per sub-block
    static constexpr int words = steps * apd;                  // activation dwords per sub-block and row

    // Activation dwords of sub-block b of stripe s for rows m0 .. m0+MT-1.
    //   W8A32: fp32 k = 128s + 4d + 2(w&1) + {0,1}, d = 2t + (w>>1)
    //   W8A16: the bf16 pair holding those two k
    //   W4A16: chunk t, k0 = 256s + 16t + 8(w>>1): the bf16 pairs at k0 + {0,4}
    //          (even w) or k0 + {2,6} (odd w)
    static __device__ __forceinline__ void load_act(uint32_t (&act)[MT][words], const cu32 *A, size_t row_dw, int s,
                                                    int b, int par, int sub_) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const cu32 *a = A + (size_t)m * row_dw;
#pragma unroll
            for (int tt = 0; tt < steps; ++tt) {
                const int t = b * steps + tt;
                if constexpr (FMT == F_W8A32) {
                    const size_t k = (size_t)s * 128 + 8 * t + 4 * par + 2 * sub_;
                    act[m][2 * tt] = a[k];
                    act[m][2 * tt + 1] = a[k + 1];
                } else if constexpr (FMT == F_W8A16) {
                    act[m][tt] = a[(size_t)s * 64 + 4 * t + 2 * par + sub_];
                } else {
                    const size_t dw = (size_t)s * 128 + 8 * t + 4 * par + sub_;
                    act[m][2 * tt] = a[dw];
                    act[m][2 * tt + 1] = a[dw + 2];
                }
            }
        }
    }
};

__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <int D>
__device__ __forceinline__ void wait_ring(bool tail) {
    if (tail)
        wait_vmcnt<0>();
    else
        wait_vmcnt<2 * (D - 2)>();
}

// The stripe loop of one wave; SUB = w & 1 selects the bytes (int8) or the
// nibble pairs (int4) of each dword, so that selection costs no instruction.
template <int FMT, int MT, int D, int SUB, int CH, int ROWS>
__device__ __forceinline__ void rows_loop(float (&acc)[MT][CH], unsigned char *lds,
                                          const uint8_t *const (&src)[2], const uint32_t (&off)[8], const cu32 *A,
                                          size_t row_dw, int ns, int wave, int par) {
    using R = RowPlan<FMT, MT>;
    constexpr int kInst = ROWS / 8;                 // DMA instructions per stripe
    constexpr int kSlot = ROWS * kStripe;
    const int nmine = (wave < kInst) + (wave + 4 < kInst);   // this wave's share: i = wave, wave + 4
    auto issue = [&](int st) {
        unsigned char *slot = lds + (st % D) * kSlot;
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
            if (wave + 4 * ii < kInst)
                __builtin_amdgcn_global_load_lds((const void *)(src[ii] + (size_t)st * kStripe),
                                                 (lds_void *)(slot + (wave + 4 * ii) * 1024), 16, 0, kNT);
    };
#pragma unroll
    for (int t = 0; t < D - 1; ++t)
        if (t < ns) issue(t);
    const uint32_t magic = opaque_magic();

    for (int s = 0; s < ns; ++s) {
        // this wave's part of stripe s has landed (its later stripes may fly)
        if (s + D - 2 >= ns || nmine == 0)
            wait_vmcnt<0>();
        else if (nmine == 1)
            wait_vmcnt<D - 2>();
        else
            wait_vmcnt<2 * (D - 2)>();
        lds_barrier();
        if (s + D - 1 < ns) issue(s + D - 1);
        uint32_t x[16];
        const unsigned char *slot = lds + (s % D) * kSlot;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            x[2 * j] = *(const uint32_t *)(slot + off[j]);
            x[2 * j + 1] = *(const uint32_t *)(slot + off[j] + 8);
        }
#pragma unroll
        for (int b = 0; b < R::sub; ++b) {
            uint32_t a[MT][R::words];
            R::load_act(a, A, row_dw, s, b, par, SUB);
            // all loads of this block are issued before any use: one wait
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int tt = 0; tt < R::steps; ++tt) {
                const uint32_t w = x[b * R::steps + tt];
                if constexpr (R::w8) {
                    const float w0 = (float)(int)(int8_t)(uint8_t)(w >> (16 * SUB));
                    const float w1 = (float)(int)(int8_t)(uint8_t)(w >> (16 * SUB + 8));
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        float a0, a1;
                        if constexpr (FMT == F_W8A32) {
                            a0 = __uint_as_float(a[m][2 * tt]);
                            a1 = __uint_as_float(a[m][2 * tt + 1]);
                        } else {
                            a0 = bf16_lo(a[m][tt]);
                            a1 = bf16_hi(a[m][tt]);
                        }
                        acc[m][0] = __builtin_fmaf(a0, w0, acc[m][0]);
                        acc[m][1] = __builtin_fmaf(a1, w1, acc[m][1]);
                    }
                } else {
                    // two exact fp16 nibble pairs of this dword (see dequant_w4)
                    const uint32_t u = w ^ 0x88888888u;
                    const uint32_t v = SUB ? (u >> 8) : u;
                    const h2 bias = {(_Float16)-1032.0f, (_Float16)-1032.0f};
                    const h2 sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
                    const h2 bias16 = {(_Float16)-72.0f, (_Float16)-72.0f};
                    const h2 qa = __builtin_bit_cast(h2, (v & 0x000F000Fu) | magic) + bias;
                    const h2 qb = __builtin_bit_cast(h2, (v & 0x00F000F0u) | magic) * sixteenth + bias16;
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        const uint32_t p0 = a[m][2 * tt], p1 = a[m][2 * tt + 1];
                        acc[m][0] = __builtin_fmaf(bf16_lo(p0), (float)qa.x, acc[m][0]);   // chain 0 / 2
                        acc[m][1] = __builtin_fmaf(bf16_lo(p1), (float)qa.y, acc[m][1]);   // chain 4 / 6
                        acc[m][2] = __builtin_fmaf(bf16_hi(p0), (float)qb.x, acc[m][2]);   // chain 1 / 3
                        acc[m][3] = __builtin_fmaf(bf16_hi(p1), (float)qb.y, acc[m][3]);   // chain 5 / 7
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// The greedy argmax epilogue (kernels.c:658-737): the bf16 logits become
// (value, index) pairs reduced in the reference scan's order -- a larger
// value first, then the lower index, from (-inf, 0) -- within the workgroup,
// parked per workgroup (part[2b], part[2b + 1]), and the last workgroup to
// take a ticket reduces the parked pairs into result[0..1] and, when not
// null, *out_index / *out_value; it leaves the ticket at zero.
struct RowsArgmax {
    uint32_t *part = nullptr;
    int *ticket = nullptr;
    uint32_t *result = nullptr;
    size_t *out_index = nullptr;
    float *out_value = nullptr;
};

__device__ __forceinline__ void rows_arg_take(float v, uint32_t n, float &bv, uint32_t &bn) {
    if (v > bv || (v == bv && n < bn)) {
        bv = v;
        bn = n;
    }
}

__device__ __forceinline__ void rows_arg_wave(float &bv, uint32_t &bn) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const uint32_t on = (uint32_t)__shfl_xor((int)bn, off);
        rows_arg_take(ov, on, bv, bn);
    }
}

template <int FMT, int MT, int D, int ROWS, bool ARG = false>
__global__ __launch_bounds__(64 * kRowWaves) void gemv_rows_kernel(const void *__restrict__ A_,
                                                                  const uint8_t *__restrict__ W,
                                                                  const float *__restrict__ S, void *__restrict__ C,
                                                                  int M, int N, int K, int m0, RowsArgmax ao) {
    static_assert(!ARG || (FMT == F_W8A16 && MT == 1), "argmax epilogue: W8A16, one activation row");
    using R = RowPlan<FMT, MT>;
    extern __shared__ __align__(16) unsigned char lds[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int row = lane & (ROWS - 1);        // lanes beyond ROWS repeat rows and write nothing
    const int par = wave >> 1, sub = wave & 1;
    const int row0 = blockIdx.x * ROWS;
    const int n = row0 + row;
    const size_t row_bytes = R::w8 ? (size_t)K : (size_t)K / 2;
    const int ns = (int)(row_bytes / kStripe);
    const size_t row_dw = FMT == F_W8A32 ? (size_t)K : (size_t)K / 2;   // activation dwords per row
    const cu32 *A = as_const(A_) + (size_t)m0 * row_dw;

    // This wave's DMA instructions per stripe: i = w and w + 4 (those below
    // ROWS / 8), each fetching rows 8i + lane/8, chunk (lane & 7) ^ ((row >> 1) & 7).
    const uint8_t *src[2];
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
        const int r = (8 * (wave + 4 * ii) + (lane >> 3)) & (ROWS - 1);
        const int q = (lane & 7) ^ ((r >> 1) & 7);
        src[ii] = W + (size_t)min(row0 + r, N - 1) * row_bytes + q * 16;
    }
    // Byte offsets of the lane's dwords in a slot: row `row`, chunk j stored at
    // position j ^ ((row >> 1) & 7); this wave reads words par and 2 + par.
    const int swz = (row >> 1) & 7;
    uint32_t off[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) off[j] = row * kStripe + ((j ^ swz) << 4) + 4 * par;

    float acc[MT][R::chains];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int c = 0; c < R::chains; ++c) acc[m][c] = 0.0f;
    if (sub)
        rows_loop<FMT, MT, D, 1, R::chains, ROWS>(acc, lds, src, off, A, row_dw, ns, wave, par);
    else
        rows_loop<FMT, MT, D, 0, R::chains, ROWS>(acc, lds, src, off, A, row_dw, ns, wave, par);

    // The chains meet in LDS (the ring is free once every wave is past its
    // last stripe): ex[chain][m][64], 8 chains for int8, 16 (lo then hi) for int4.
    float *ex = (float *)lds;
    lds_barrier();
#pragma unroll
    for (int c = 0; c < R::chains; ++c) {
        int chain;
        if constexpr (R::w8) {
            chain = 4 * par + 2 * sub + c;
        } else {
            const int lo_ids[4] = {0, 4, 1, 5};
            chain = 8 * par + lo_ids[c] + 2 * sub;
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) ex[(chain * MT + m) * 64 + lane] = acc[m][c];
    }
    __syncthreads();
    if constexpr (ARG) {
        // wave 0: this tile's best pair, parked; the workgroup that takes the
        // last ticket reduces every parked pair with all its threads
        // (in the dynamic LDS past the 8 x 64 chain sums: a static array would
        // count against the 160 KB the launch raises the dynamic limit to)
        int &s_last = *(int *)(ex + 8 * 64);
        float *s_v = ex + 8 * 64 + 4;
        uint32_t *s_n = (uint32_t *)(ex + 8 * 64 + 4 + kRowWaves);
        if (wave == 0) {
            float bv = -__builtin_inff();
            uint32_t bn = 0;
            if (lane < ROWS && n < N) {
                float l[8];
#pragma unroll
                for (int c = 0; c < 8; ++c) l[c] = ex[c * 64 + lane];
                const float y = hsum8(l) * S[n];
                rows_arg_take(__uint_as_float((uint32_t)f32_to_bf16(y) << 16), (uint32_t)n, bv, bn);
            }
            rows_arg_wave(bv, bn);
            if (lane == 0) {
                // agent-scope stores reach the device-coherent level; once
                // they have completed the lane takes a ticket (no cache-wide
                // release: that writes back a whole L2 per workgroup)
                __hip_atomic_store(ao.part + 2 * blockIdx.x, __float_as_uint(bv), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(ao.part + 2 * blockIdx.x + 1, bn, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                wait_vmcnt<0>();
                const int tk = __hip_atomic_fetch_add(ao.ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s_last = tk == (int)gridDim.x - 1;
            }
        }
        __syncthreads();
        if (!s_last) return;
        float bv = -__builtin_inff();
        uint32_t bn = 0;
        const uint32_t t = threadIdx.x;
        // every thread's pairs loaded before any is compared (the loads are
        // independent; one round trip instead of one per pair)
        constexpr int kPer = 16;
        for (uint32_t b0 = t; b0 < gridDim.x; b0 += kPer * 64 * kRowWaves) {
            uint32_t v[kPer], i[kPer];
#pragma unroll
            for (int u = 0; u < kPer; ++u) {
                const uint32_t b = b0 + (uint32_t)u * 64 * kRowWaves;
                if (b < gridDim.x) {
                    v[u] = __hip_atomic_load(ao.part + 2 * b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    i[u] = __hip_atomic_load(ao.part + 2 * b + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
#pragma unroll
            for (int u = 0; u < kPer; ++u)
                if (b0 + (uint32_t)u * 64 * kRowWaves < gridDim.x) rows_arg_take(__uint_as_float(v[u]), i[u], bv, bn);
        }
        rows_arg_wave(bv, bn);
        if (lane == 0) {
            s_v[wave] = bv;
            s_n[wave] = bn;
        }
        __syncthreads();
        if (t == 0) {
            for (int w = 1; w < kRowWaves; ++w) rows_arg_take(s_v[w], s_n[w], bv, bn);
            ao.result[0] = __float_as_uint(bv);
            ao.result[1] = bn;
            if (ao.out_index) *ao.out_index = (size_t)bn;
            if (ao.out_value) *ao.out_value = bv;
            __hip_atomic_store(ao.ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    if (wave != 0 || lane >= ROWS || n >= N) return;
    const float scale = S[n];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        float l[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            l[c] = ex[(c * MT + m) * 64 + lane];
            if constexpr (!R::w8) l[c] = l[c] + ex[((8 + c) * MT + m) * 64 + lane];
        }
        const float y = hsum8(l) * scale;
        const size_t o = (size_t)(m0 + m) * N + n;
        if constexpr (FMT == F_W8A32)
            ((float *)C)[o] = y;
        else
            ((uint16_t *)C)[o] = f32_to_bf16(y);
    }
}

constexpr size_t kRowMaxLds = 160 * 1024;

template <int FMT, int MT, int D, int ROWS>
int launch_rows_one(hipStream_t st, const void *A, const uint8_t *W, const float *S, void *C, int M, int N, int K,
                    int m0) {
    static std::once_flag once;
    static hipError_t attr_rc = hipSuccess;
    std::call_once(once, [] {
        attr_rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_rows_kernel<FMT, MT, D, ROWS>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRowMaxLds);
    });
    if (attr_rc != hipSuccess) return ECPU_ERR_DEVICE;
    const size_t lds = std::max<size_t>((size_t)D * ROWS * kStripe, (size_t)16 * MT * 64 * sizeof(float));
    const dim3 grid((unsigned)((N + ROWS - 1) / ROWS));
    gemv_rows_kernel<FMT, MT, D, ROWS><<<grid, 64 * kRowWaves, lds, st>>>(A, W, S, C, M, N, K, m0, RowsArgmax{});
    return ECPU_OK;
}

template <int D, int ROWS>
int launch_rows_argmax(hipStream_t st, const uint16_t *A, const uint8_t *W, const float *S, int N, int K,
                       const RowsArgmax &ao) {
    static std::once_flag once;
    static hipError_t attr_rc = hipSuccess;
    std::call_once(once, [] {
        attr_rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_rows_kernel<F_W8A16, 1, D, ROWS, true>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRowMaxLds);
    });
    if (attr_rc != hipSuccess) return ECPU_ERR_DEVICE;
    const size_t lds = std::max<size_t>((size_t)D * ROWS * kStripe, (size_t)16 * 64 * sizeof(float));
    const dim3 grid((unsigned)((N + ROWS - 1) / ROWS));
    gemv_rows_kernel<F_W8A16, 1, D, ROWS, true><<<grid, 64 * kRowWaves, lds, st>>>(A, W, S, nullptr, 1, N, K, 0, ao);
    return ECPU_OK;
}

template <int FMT, int D, int ROWS>
int launch_rows_mt(int mt, hipStream_t st, const void *A, const uint8_t *W, const float *S, void *C, int M, int N,
                   int K, int m0) {
    switch (mt) {
        case 1: return launch_rows_one<FMT, 1, D, ROWS>(st, A, W, S, C, M, N, K, m0);
        case 2: return launch_rows_one<FMT, 2, D, ROWS>(st, A, W, S, C, M, N, K, m0);
        case 3: return launch_rows_one<FMT, 3, D, ROWS>(st, A, W, S, C, M, N, K, m0);
        default: return launch_rows_one<FMT, 4, D, ROWS>(st, A, W, S, C, M, N, K, m0);
    }
}

template <int FMT>
int launch_rows_fmt(int rows, int depth, int mt, hipStream_t st, const void *A, const uint8_t *W, const float *S,
                    void *C, int M, int N, int K, int m0) {
    if (rows == 16) return launch_rows_mt<FMT, 16, 16>(mt, st, A, W, S, C, M, N, K, m0);
    if (rows == 32) return launch_rows_mt<FMT, 16, 32>(mt, st, A, W, S, C, M, N, K, m0);
    switch (depth) {
        case 16: return launch_rows_mt<FMT, 16, 64>(mt, st, A, W, S, C, M, N, K, m0);
        case 8: return launch_rows_mt<FMT, 8, 64>(mt, st, A, W, S, C, M, N, K, m0);
        default: return launch_rows_mt<FMT, 4, 64>(mt, st, A, W, S, C, M, N, K, m0);
    }
}

// ------------------------------------------------------------------ quad
// A CU streams only ~25-30 GB/s however deep its prefetch, so a GEMV must
// spread over all CUs; 64-row tiles leave most of them idle when N is a few
// thousand rows.  The quad kernel uses 16-row tiles: lane = 4r + c serves row
// r of the tile with chain group c = lane & 3,
//   int8: chains {2c, 2c+1} = bytes 2(c&1), 2(c&1)+1 of the dwords of parity
//         c >> 1 (k = 8T + 2c + {0,1});
//   int4: the lo (c < 2) or hi (c >= 2) chains of each chunk, nibble pairs
//         (0,4),(1,5) for even c and (2,6),(3,7) for odd c;
// and the four partial chain sets of a row meet through DPP quad permutes in
// the reference's hsum order.  The activations of a chain group are not the
// same for all lanes any more, so each workgroup first copies its activation
// rows into LDS (global -> LDS DMA) and every lane reads its own words:
//   W8A32  fp32 a[8T + 2c], a[8T + 2c + 1]            (T = k / 8)
//   W8A16  the bf16 pair dword 4T + c
//   W4A16  the bf16 pair dwords 8T + 4(c>>1) + (c&1) + {0, 2}   (T = k / 16)
// Each wave owns a 16-row tile and its own ring of D stripe slots (16 rows x
// 128 B, two DMA instructions per stripe), so no barrier is needed per stripe.

constexpr int kQuadSlotBytes = 16 * kStripe;   // one stripe: 16 rows x 128 B

template <int FMT>
struct QuadFmt {
    static constexpr bool w8 = FMT != F_W4ROW;
    static constexpr int chains = w8 ? 2 : 4;
    static constexpr int apd = FMT == F_W8A16 ? 1 : 2;   // activation dwords per lane and step
    // activation dwords per row
    static __device__ __forceinline__ int row_dw(int K) { return FMT == F_W8A32 ? K : K / 2; }
    // first activation dword of step T for chain group c; the second one
    // (apd 2) follows at +1 (fp32) or +2 (bf16 pairs of int4 nibble pairs)
    static __device__ __forceinline__ int act_index(int T, int c) {
        if constexpr (FMT == F_W8A32)
            return 8 * T + 2 * c;
        else if constexpr (FMT == F_W8A16)
            return 4 * T + c;
        else
            return 8 * T + 4 * (c >> 1) + (c & 1);
    }
    static constexpr int second = FMT == F_W8A32 ? 1 : 2;
};

__device__ __forceinline__ float dpp_quad_add(float x, int ctrl_is_swap2) {
    // x + x of the partner lane in the quad: [2,3,0,1] (ctrl 0x4E) or [1,0,3,2] (0xB1)
    const int xi = __builtin_bit_cast(int, x);
    const int y = ctrl_is_swap2 ? __builtin_amdgcn_update_dpp(0, xi, 0x4E, 0xF, 0xF, false)
                                : __builtin_amdgcn_update_dpp(0, xi, 0xB1, 0xF, 0xF, false);
    return x + __builtin_bit_cast(float, y);
}

// SW: the SwiGLU variant of the W4 per-row kernel (kernels.c:1598-1659).  W
// holds 2N rows (gate rows 0..N-1, then the up rows), and tile t covers gate
// rows 8t..8t+7 (lanes 0-31) with their up rows N+8t..N+8t+7 (lanes 32-63);
// the epilogue writes C[i] = bf16(silu(g) * u) for the N gate rows.
template <int FMT, int MT, int D, bool SW = false>
__global__ __launch_bounds__(256) void gemv_quad_kernel(const void *__restrict__ A_, const uint8_t *__restrict__ W,
                                                       const float *__restrict__ S, void *__restrict__ C, int M,
                                                       int N, int K, int m0, int ntiles) {
    using Q = QuadFmt<FMT>;
    static_assert(!SW || (FMT == F_W4ROW && MT == 1), "SwiGLU epilogue: W4 per-row, one activation row");
    extern __shared__ __align__(16) unsigned char lds[];
    const int wpb = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int r = lane >> 2, c = lane & 3, par = c >> 1;
    const int tile = blockIdx.x * wpb + wave;
    const int row0 = tile * 16;
    const size_t row_bytes = Q::w8 ? (size_t)K : (size_t)K / 2;
    const int ns = (int)(row_bytes / kStripe);
    const int rdw = Q::row_dw(K);
    unsigned char *act = lds + (size_t)wpb * D * kQuadSlotBytes;

    // Activation rows m0 .. m0+MT-1 (contiguous in A) into LDS: 16-byte DMA,
    // 256 dwords per instruction, instructions dealt round-robin to the waves.
    {
        const int total = MT * rdw;
        const uint32_t *a = (const uint32_t *)A_ + (size_t)m0 * rdw;
        int issued = 0;
        for (int q = wave; q * 256 < total; q += wpb) {
            const int g = q * 256 + 4 * lane;
            if (g < total)
                __builtin_amdgcn_global_load_lds((const void *)(a + g), (lds_void *)(act + (size_t)q * 1024), 16, 0,
                                                 0);
            if ((++issued & 15) == 0) wait_vmcnt<16>();   // keep the wave's outstanding loads bounded
        }
    }

    // This wave's stripe DMA: instruction i fetches rows 8i + lane/8 of the
    // tile, chunk (lane & 7) ^ ((row >> 1) & 7).
    const uint8_t *src[2];
    const bool live = tile < ntiles;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int rr = 8 * i + (lane >> 3);
        const int q = (lane & 7) ^ ((rr >> 1) & 7);
        const size_t wrow = SW ? (size_t)(i ? N : 0) + (size_t)min(8 * tile + (rr & 7), N - 1)
                               : (size_t)min(row0 + rr, N - 1);
        src[i] = W + wrow * row_bytes + q * 16;
    }
    unsigned char *ring = lds + (size_t)wave * D * kQuadSlotBytes;
    auto issue = [&](int st) {
        unsigned char *slot = ring + (st % D) * kQuadSlotBytes;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(src[i] + (size_t)st * kStripe),
                                             (lds_void *)(slot + i * 1024), 16, 0, kNT);
    };
    if (live) {
#pragma unroll
        for (int t = 0; t < D - 2; ++t)
            if (t < ns) issue(t);
    }
    // This wave's activation copies are older than its (at most 2(D-2))
    // stripe loads; after the barrier every wave's copies have landed.
    if (live && ns >= D - 2)
        wait_vmcnt<2 * (D - 2)>();
    else
        wait_vmcnt<0>();
    asm volatile("s_barrier" ::: "memory");
    if (!live) return;

    // Lane's word offsets in a slot: row r, chunk j at position j ^ ((r >> 1) & 7),
    // words par and par + 2.
    const int swz = (r >> 1) & 7;
    uint32_t off[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) off[j] = r * kStripe + ((j ^ swz) << 4) + 4 * par;
    const uint32_t *my_act = (const uint32_t *)act + Q::act_index(0, c);
    const uint32_t shift = Q::w8 ? 16u * (c & 1) : 8u * (c & 1);
    const uint32_t magic = opaque_magic();

    float acc[MT][Q::chains];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int k = 0; k < Q::chains; ++k) acc[m][k] = 0.0f;

    // One stripe's words (x) and activations (av) for the lane.
    auto load = [&](int st, uint32_t (&x)[16], uint32_t (&av)[MT][16 * Q::apd]) {
        const unsigned char *slot = ring + (st % D) * kQuadSlotBytes;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            x[2 * j] = *(const uint32_t *)(slot + off[j]);
            x[2 * j + 1] = *(const uint32_t *)(slot + off[j] + 8);
        }
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const uint32_t *ap = my_act + (size_t)m * rdw + Q::act_index(16 * st + t, 0);
                if constexpr (Q::apd == 2) {
                    av[m][2 * t] = ap[0];
                    av[m][2 * t + 1] = ap[Q::second];
                } else {
                    av[m][t] = ap[0];
                }
            }
    };
    auto compute = [&](const uint32_t (&x)[16], const uint32_t (&av)[MT][16 * Q::apd]) {
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const uint32_t w = x[t];
            if constexpr (Q::w8) {
                const uint32_t ws = w >> shift;
                const float w0 = (float)(int)(int8_t)(uint8_t)ws;
                const float w1 = (float)(int)(int8_t)(uint8_t)(ws >> 8);
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    float a0, a1;
                    if constexpr (FMT == F_W8A32) {
                        a0 = __uint_as_float(av[m][2 * t]);
                        a1 = __uint_as_float(av[m][2 * t + 1]);
                    } else {
                        a0 = bf16_lo(av[m][t]);
                        a1 = bf16_hi(av[m][t]);
                    }
                    acc[m][0] = __builtin_fmaf(a0, w0, acc[m][0]);
                    acc[m][1] = __builtin_fmaf(a1, w1, acc[m][1]);
                }
            } else {
                const uint32_t v = (w ^ 0x88888888u) >> shift;
                const h2 bias = {(_Float16)-1032.0f, (_Float16)-1032.0f};
                const h2 sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
                const h2 bias16 = {(_Float16)-72.0f, (_Float16)-72.0f};
                const h2 qa = __builtin_bit_cast(h2, (v & 0x000F000Fu) | magic) + bias;
                const h2 qb = __builtin_bit_cast(h2, (v & 0x00F000F0u) | magic) * sixteenth + bias16;
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const uint32_t p0 = av[m][2 * t], p1 = av[m][2 * t + 1];
                    acc[m][0] = __builtin_fmaf(bf16_lo(p0), (float)qa.x, acc[m][0]);   // chain 0 / 2
                    acc[m][1] = __builtin_fmaf(bf16_lo(p1), (float)qa.y, acc[m][1]);   // chain 4 / 6
                    acc[m][2] = __builtin_fmaf(bf16_hi(p0), (float)qb.x, acc[m][2]);   // chain 1 / 3
                    acc[m][3] = __builtin_fmaf(bf16_hi(p1), (float)qb.y, acc[m][3]);   // chain 5 / 7
                }
            }
        }
    };
    // Software pipeline, two stripes per round: while stripe s is computed
    // from registers, stripe s+1 is read from LDS (LDS reads complete in
    // order, so only the reads of s+1 are waited for, when they are used).
    // Slots are refilled only at the top of a round, with the stripes of the
    // two slots consumed in the previous round, so no DMA can overtake a read
    // of its slot; D-2 stripes stay in flight.
    uint32_t xa[16], xb[16];
    uint32_t aa[MT][16 * Q::apd], ab[MT][16 * Q::apd];
    if (ns >= D - 2)
        wait_vmcnt<2 * (D - 3)>();   // stripe 0 of the D-2 issued
    else
        wait_vmcnt<0>();
    load(0, xa, aa);
    int s = 0;
    for (; s + 1 < ns; s += 2) {
        if (s + D - 2 < ns) issue(s + D - 2);   // slot of stripe s-2
        if (s + D - 1 < ns) issue(s + D - 1);   // slot of stripe s-1
        if (s + D <= ns)
            wait_vmcnt<2 * (D - 2)>();          // stripe s+1 (s+2 .. s+D-1 may fly)
        else
            wait_vmcnt<0>();
        load(s + 1, xb, ab);
        compute(xa, aa);
        if (s + 2 < ns) {
            if (s + D <= ns)
                wait_vmcnt<2 * (D - 3)>();      // stripe s+2 (s+3 .. s+D-1 may fly)
            else
                wait_vmcnt<0>();
            load(s + 2, xa, aa);
        }
        compute(xb, ab);
    }
    if (s < ns) compute(xa, aa);


    // Reference order of the 8-lane horizontal sum (int4: of lo[l] + hi[l]):
    //   ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)).
    // int8: c holds (l_{2c}, l_{2c+1}); c ^ 2 holds (l_{2c+4}, l_{2c+5}).
    // int4: c holds lo (c < 2) or hi (c >= 2) of chains {0,4,1,5} (even c) or
    //       {2,6,3,7} (odd c); c ^ 2 holds the other half of the same chains.
    const int n = row0 + r;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        float h;
        if constexpr (Q::w8) {
            const float p0 = dpp_quad_add(acc[m][0], 1);   // l_{2c} + l_{2c+4}
            const float p1 = dpp_quad_add(acc[m][1], 1);   // l_{2c+1} + l_{2c+5}
            h = dpp_quad_add(p0 + p1, 0);                   // c = 0: (l0+l4)+(l1+l5) + (l2+l6)+(l3+l7)
        } else {
            const float s0 = dpp_quad_add(acc[m][0], 1);   // s0 / s2  (lo + hi)
            const float s4 = dpp_quad_add(acc[m][1], 1);   // s4 / s6
            const float s1 = dpp_quad_add(acc[m][2], 1);   // s1 / s3
            const float s5 = dpp_quad_add(acc[m][3], 1);   // s5 / s7
            h = dpp_quad_add((s0 + s4) + (s1 + s5), 0);
        }
        if constexpr (SW) {
            // up-row sums of lanes 32-63 meet the gate-row sums of lanes 0-31
            const float hu = __shfl_xor(h, 32);
            const int i = 8 * tile + r;
            if (lane < 32 && c == 0 && i < N) {
                const float g = __uint_as_float((uint32_t)f32_to_bf16(h * S[i]) << 16);
                const float u = __uint_as_float((uint32_t)f32_to_bf16(hu * S[N + i]) << 16);
                ((uint16_t *)C)[(size_t)(m0 + m) * N + i] = swiglu_bf16_value(g, u);
            }
        } else if (c == 0 && n < N) {
            const float y = h * S[n];
            const size_t o = (size_t)(m0 + m) * N + n;
            if constexpr (FMT == F_W8A32)
                ((float *)C)[o] = y;
            else
                ((uint16_t *)C)[o] = f32_to_bf16(y);
        }
    }
}

template <int FMT, int MT, int D, bool SW = false>
int launch_quad_one(int wpb, int ntiles, hipStream_t st, const void *A, const uint8_t *W, const float *S, void *C,
                    int M, int N, int K, int m0) {
    static std::once_flag once;
    static hipError_t attr_rc = hipSuccess;
    std::call_once(once, [] {
        attr_rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_quad_kernel<FMT, MT, D, SW>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRowMaxLds);
    });
    if (attr_rc != hipSuccess) return ECPU_ERR_DEVICE;
    const size_t rdw = FMT == F_W8A32 ? (size_t)K : (size_t)K / 2;
    const size_t lds = (size_t)wpb * D * kQuadSlotBytes + (size_t)MT * rdw * 4;
    if (lds > kRowMaxLds) return ECPU_ERR_UNSUPPORTED;
    const dim3 grid((unsigned)((ntiles + wpb - 1) / wpb));
    gemv_quad_kernel<FMT, MT, D, SW><<<grid, 64 * wpb, lds, st>>>(A, W, S, C, M, N, K, m0, ntiles);
    return ECPU_OK;
}

template <int FMT, int D>
int launch_quad_mt(int mt, int wpb, int ntiles, hipStream_t st, const void *A, const uint8_t *W, const float *S,
                   void *C, int M, int N, int K, int m0) {
    switch (mt) {
        case 1: return launch_quad_one<FMT, 1, D>(wpb, ntiles, st, A, W, S, C, M, N, K, m0);
        case 2: return launch_quad_one<FMT, 2, D>(wpb, ntiles, st, A, W, S, C, M, N, K, m0);
        case 3: return launch_quad_one<FMT, 3, D>(wpb, ntiles, st, A, W, S, C, M, N, K, m0);
        default: return launch_quad_one<FMT, 4, D>(wpb, ntiles, st, A, W, S, C, M, N, K, m0);
    }
}

template <int FMT>
int launch_quad_fmt(int depth, int mt, int wpb, int ntiles, hipStream_t st, const void *A, const uint8_t *W,
                    const float *S, void *C, int M, int N, int K, int m0) {
    switch (depth) {
        case 16: return launch_quad_mt<FMT, 16>(mt, wpb, ntiles, st, A, W, S, C, M, N, K, m0);
        case 8: return launch_quad_mt<FMT, 8>(mt, wpb, ntiles, st, A, W, S, C, M, N, K, m0);
        default: return launch_quad_mt<FMT, 4>(mt, wpb, ntiles, st, A, W, S, C, M, N, K, m0);
    }
}

// ------------------------------------------------------------------ chain
// With few 16-row tiles (a few thousand rows and a long K: o_proj, down) the
// quad kernel runs one wave per tile, i.e. on one SIMD of a CU, and is VALU
// bound.  The chain kernel gives each 16-row tile CS waves (CS SIMDs of one
// CU) and divides the quad lane's chains among them, so every lane carries
// fewer chains:
//   int4: CS = 4 (one chain per lane) or 2; lane (r, c) of wave w owns slots
//         g = w * (4/CS) + i of chain group c, nibble 2(c&1) + (g>>1) + 4(g&1)
//         of the dwords of parity c>>1 -- the quad kernel's chains
//         {0,4,1,5} / {2,6,3,7} of the lo (c < 2) or hi half;
//   int8: CS = 2; wave w owns byte 2(c&1) + w of the dwords of parity c>>1
//         (chain 2c + w).
// A weight is decoded with one sign-extending bit-field extract and one
// conversion.  Each workgroup first converts its activation rows to fp32 in
// LDS, laid out chain by chain (the 16 values a chain meets in one stripe are
// contiguous), so a lane reads them with four 16-byte loads that every lane of
// the chain shares.  The waves share one ring of D stripe slots (waves 0 and
// 1 issue a stripe's two DMA instructions) with one barrier per stripe; at
// the end the chain sums meet in LDS and one lane per row adds them in the
// reference's order.
template <int FMT, int CS>
struct ChainFmt {
    static constexpr bool w8 = FMT != F_W4ROW;
    static constexpr int nchain = w8 ? 8 : 16;     // chains per row
    static constexpr int gslots = w8 ? 2 : 4;      // chain slots of a lane group, all waves
    static constexpr int slots = gslots / CS;      // chain slots per lane
    static_assert(slots >= 1 && gslots % CS == 0, "chain split");
    static constexpr int width = w8 ? 8 : 4;       // bits per weight
    static __device__ __forceinline__ int bit(int c, int g) {
        return w8 ? 8 * (2 * (c & 1) + g) : 4 * (2 * (c & 1) + (g >> 1) + 4 * (g & 1));
    }
    static __device__ __forceinline__ int chain(int c, int g) {
        return w8 ? 4 * (c >> 1) + 2 * (c & 1) + g : 8 * (c >> 1) + 2 * (c & 1) + (g >> 1) + 4 * (g & 1);
    }
    // Position of activation k in the chain-major layout: stripe s, chain,
    // then the chain's 16 values of the stripe in the lane's word order
    // t = 2j + qq (chunk j, dword q = parity + 2qq).  Blocks are kBlock = 20
    // floats apart (16 used): the four chain groups of a wave then read
    // different LDS banks (a 16-float pitch put two of them on the same banks).
    static constexpr int kBlock = 20;
    static __device__ __forceinline__ int row_floats(int K) { return K / 16 * kBlock; }
    static __device__ __forceinline__ int perm(int k) {
        if constexpr (w8) {
            const int s = k >> 7, j = (k >> 4) & 7, q = (k >> 2) & 3, b = k & 3;
            return (s * 8 + 4 * (q & 1) + b) * kBlock + 2 * j + (q >> 1);
        } else {
            const int s = k >> 8, j = (k >> 5) & 7, q = (k >> 3) & 3, p = k & 7;
            return (s * 16 + 8 * (q & 1) + p) * kBlock + 2 * j + (q >> 1);
        }
    }
};

__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int FMT, int MT, int D, int CS>
__global__ __launch_bounds__(256) void gemv_chain_kernel(const void *__restrict__ A_, const uint8_t *__restrict__ W,
                                                        const float *__restrict__ S, void *__restrict__ C, int N,
                                                        int K, int m0) {
    using F = ChainFmt<FMT, CS>;
    extern __shared__ __align__(16) unsigned char lds[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int r = lane >> 2, c = lane & 3, par = c >> 1;
    const int row0 = blockIdx.x * 16;
    const size_t row_bytes = F::w8 ? (size_t)K : (size_t)K / 2;
    const int ns = (int)(row_bytes / kStripe);
    unsigned char *ring = lds;
    constexpr int kEbytes = FMT == F_W8A32 ? 4 : 2;   // bytes per activation
    float *act = (float *)(lds + (size_t)D * kQuadSlotBytes);
    const int arow = F::row_floats(K);   // floats per activation row in LDS
    float *red = act + (size_t)MT * arow;

    // Stripe DMA: instruction i (issued by wave i, i < 2) fetches rows
    // 8i + lane/8 of the tile, chunk (lane & 7) ^ ((row >> 1) & 7).
    const bool issuer = wave < 2;
    const int ii = wave & 1;
    const int rr = 8 * ii + (lane >> 3);
    const uint8_t *src = W + (size_t)min(row0 + rr, N - 1) * row_bytes + (((lane & 7) ^ ((rr >> 1) & 7)) << 4);
    auto issue = [&](int st) {
        __builtin_amdgcn_global_load_lds((const void *)(src + (size_t)st * kStripe),
                                         (lds_void *)(ring + (st % D) * kQuadSlotBytes + ii * 1024), 16, 0, kNT);
    };
    // Rounds of R stripes: the issuers keep D - R stripes in flight; a round
    // starts once its R stripes have landed (and, by the barrier, once every
    // wave is done with the previous round, whose slots then take the next R
    // stripes).  Within a round the LDS reads of stripe u+1 are issued before
    // stripe u is computed.  Rounds are complete (no branch inside, so each
    // compute waits only for its own reads); a tail of ns % R stripes follows.
    constexpr int R = 4;
    static_assert(D % R == 0 && D >= 2 * R, "ring depth");

    // Activation rows m0.. -> fp32, chain-major (16-byte loads, four per
    // lane in flight), then the first D - R stripes.  (Copying the
    // activations by DMA behind the stripes instead measured slower.)
    {
        constexpr int epv = 16 / kEbytes;   // elements per 16-byte vector
        const int nvec = K / epv, nthr = 64 * CS;
#pragma unroll 1
        for (int m = 0; m < MT; ++m) {
            const u32x4 *asrc = (const u32x4 *)((const unsigned char *)A_ + (size_t)(m0 + m) * K * kEbytes);
            float *dst = act + (size_t)m * arow;
#pragma unroll 1
            for (int v0 = 0; v0 < nvec; v0 += 4 * nthr) {
                u32x4 buf[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int v = v0 + u * nthr + (int)threadIdx.x;
                    if (v < nvec) buf[u] = asrc[v];
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int v = v0 + u * nthr + (int)threadIdx.x;
                    if (v >= nvec) continue;
#pragma unroll
                    for (int e = 0; e < epv; ++e) {
                        const uint32_t word = buf[u][epv == 4 ? e : e >> 1];
                        dst[F::perm(v * epv + e)] =
                            epv == 4 ? __uint_as_float(word) : ((e & 1) ? bf16_hi(word) : bf16_lo(word));
                    }
                }
            }
        }
    }
    if (issuer) {
#pragma unroll 1
        for (int t = 0; t < D - R; ++t)
            if (t < ns) issue(t);
    }
    // (the first round's barrier orders the activation writes before any read)

    const int swz = (r >> 1) & 7;
    uint32_t off[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) off[j] = r * kStripe + ((j ^ swz) << 4) + 4 * par;
    int bits[F::slots], chn[F::slots];
#pragma unroll
    for (int i = 0; i < F::slots; ++i) {
        bits[i] = F::bit(c, wave * F::slots + i);
        chn[i] = F::chain(c, wave * F::slots + i);
    }
    float acc[MT][F::slots];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int i = 0; i < F::slots; ++i) acc[m][i] = 0.0f;

    uint32_t xw[2][16];
    f32x4 av[2][MT][F::slots][4];
    auto load = [&](int s, int b) {
        const unsigned char *slot = ring + (s % D) * kQuadSlotBytes;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            xw[b][2 * j] = *(const uint32_t *)(slot + off[j]);
            xw[b][2 * j + 1] = *(const uint32_t *)(slot + off[j] + 8);
        }
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int i = 0; i < F::slots; ++i) {
                const f32x4 *ap = (const f32x4 *)(act + (size_t)m * arow + (s * F::nchain + chn[i]) * F::kBlock);
#pragma unroll
                for (int v = 0; v < 4; ++v) av[b][m][i][v] = ap[v];
            }
    };
    auto compute = [&](int b) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int i = 0; i < F::slots; ++i)
#pragma unroll
                for (int t = 0; t < 16; ++t) {
                    const float w = (float)(int)__builtin_amdgcn_sbfe((int)xw[b][t], bits[i], F::width);
                    acc[m][i] = __builtin_fmaf(av[b][m][i][t >> 2][t & 3], w, acc[m][i]);
                }
    };

    const int nfull = ns / R * R;
#pragma unroll 1
    for (int s0 = 0; s0 < nfull; s0 += R) {
        if (issuer) {
            if (s0 + D - R - 1 < ns)
                wait_vmcnt<D - 2 * R>();   // stripes s0+R .. s0+D-R-1 may still fly
            else
                wait_vmcnt<0>();
        }
        lds_sync();
        if (issuer) {
#pragma unroll
            for (int u = 0; u < R; ++u)
                if (s0 + D - R + u < ns) issue(s0 + D - R + u);
        }
        load(s0, 0);
#pragma unroll
        for (int u = 0; u < R; ++u) {
            // keep the order: reads of u, reads of u+1, then the math of u
            __builtin_amdgcn_sched_barrier(0);
            if (u + 1 < R) load(s0 + u + 1, (u + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
            compute(u & 1);
        }
    }
    // The last ns % R stripes (already issued), one at a time.
#pragma unroll 1
    for (int s = nfull; s < ns; ++s) {
        if (issuer) wait_vmcnt<0>();
        lds_sync();
        load(s, 0);
        compute(0);
    }

    // The chain sums meet in LDS; lane 4r of wave 0 adds row r's chains in
    // the reference's order: hsum ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)) of the 8
    // lanes (int4: of lo[l] + hi[l]), times the row scale.
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int i = 0; i < F::slots; ++i) red[(m * F::gslots + wave * F::slots + i) * 64 + lane] = acc[m][i];
    lds_sync();
    const int n = row0 + r;
    if (wave != 0 || c != 0 || n >= N) return;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const float *rb = red + m * F::gslots * 64 + 4 * r;
        float l8[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            if constexpr (F::w8) {
                const int b = l & 3;
                l8[l] = rb[(b & 1) * 64 + 2 * (l >> 2) + (b >> 1)];
            } else {
                const int cl = (l >> 1) & 1, gl = ((l >> 2) & 1) + 2 * (l & 1);
                l8[l] = rb[gl * 64 + cl] + rb[gl * 64 + cl + 2];
            }
        }
        const float y = hsum8(l8) * S[n];
        const size_t o = (size_t)(m0 + m) * N + n;
        if constexpr (FMT == F_W8A32)
            ((float *)C)[o] = y;
        else
            ((uint16_t *)C)[o] = f32_to_bf16(y);
    }
}

template <int FMT, int MT, int D, int CS>
size_t chain_lds_bytes(int K) {
    // ring, fp32 activations (20-float chain blocks), chain sums
    return (size_t)D * kQuadSlotBytes + (size_t)MT * (K / 16) * ChainFmt<FMT, CS>::kBlock * 4 +
           (size_t)MT * ChainFmt<FMT, CS>::gslots * 64 * 4;
}

template <int FMT, int MT, int D, int CS>
int launch_chain_one(int ntiles, hipStream_t st, const void *A, const uint8_t *W, const float *S, void *C, int N,
                     int K, int m0) {
    static std::once_flag once;
    static hipError_t attr_rc = hipSuccess;
    std::call_once(once, [] {
        attr_rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_chain_kernel<FMT, MT, D, CS>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRowMaxLds);
    });
    if (attr_rc != hipSuccess) return ECPU_ERR_DEVICE;
    const size_t lds = chain_lds_bytes<FMT, MT, D, CS>(K);
    if (lds > kRowMaxLds) return ECPU_ERR_UNSUPPORTED;
    gemv_chain_kernel<FMT, MT, D, CS><<<ntiles, 64 * CS, lds, st>>>(A, W, S, C, N, K, m0);
    return ECPU_OK;
}

template <int FMT, int CS>
int launch_chain_mt(int mt, int ntiles, hipStream_t st, const void *A, const uint8_t *W, const float *S, void *C,
                    int N, int K, int m0) {
    switch (mt) {
        case 1: return launch_chain_one<FMT, 1, 16, CS>(ntiles, st, A, W, S, C, N, K, m0);
        case 2: return launch_chain_one<FMT, 2, 16, CS>(ntiles, st, A, W, S, C, N, K, m0);
        case 3: return launch_chain_one<FMT, 3, 16, CS>(ntiles, st, A, W, S, C, N, K, m0);
        default: return launch_chain_one<FMT, 4, 16, CS>(ntiles, st, A, W, S, C, N, K, m0);
    }
}

// Activation rows per launch of the chain kernel: 4, 2 or 1, whichever is the
// largest that fits LDS (the fp32 activations take 4K bytes per row).
template <int FMT, int CS>
int chain_rows_per_launch(int K) {
    if (chain_lds_bytes<FMT, 4, 16, CS>(K) <= kRowMaxLds) return 4;
    if (chain_lds_bytes<FMT, 2, 16, CS>(K) <= kRowMaxLds) return 2;
    if (chain_lds_bytes<FMT, 1, 16, CS>(K) <= kRowMaxLds) return 1;
    return 0;
}

// ------------------------------------------------------------------ chain, 8 rows
// W4 per-row (bundle v2), one activation row, a few thousand rows: the chain
// kernel's 16-row tiles leave CUs idle below 4096 rows (k/v 1024: 64 tiles).
// Here a tile has 8 rows, lane 8r + c serves row r with chain group c (lo
// half for c < 4, hi for c >= 4; nibbles c & 3 and (c & 3) + 4) and the two
// waves of the workgroup take one of those two chains each, so every lane
// runs one chain: chain 8h + l, l = (c & 3) + 4w.  Activations are staged in
// LDS chain-major as in the chain kernel (a lane reads its chain's sixteen
// values of a stripe with four 16-byte loads shared by the eight rows); the
// waves share a ring of D one-stripe slots (wave 0 issues the DMA, one
// barrier per round of four stripes); chain sums meet in LDS and lane r of
// wave 0 adds lo[l] + hi[l], then the reference's hsum, times the scale.
template <int D>
__global__ __launch_bounds__(128) void gemv_w4c8_kernel(const uint16_t *__restrict__ A, const uint8_t *__restrict__ W,
                                                       const float *__restrict__ S, uint16_t *__restrict__ C, int N,
                                                       int K) {
    using F = ChainFmt<F_W4ROW, 4>;   // activation layout (perm, row_floats) only
    constexpr int R = 4;
    constexpr int SLOT = 8 * kStripe;
    static_assert(D % R == 0 && D >= 2 * R, "ring depth");
    extern __shared__ __align__(16) unsigned char lds[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int r = lane >> 3, c = lane & 7, par = c >> 2;
    const int l = (c & 3) + 4 * wave;      // the lane's chain within its half
    const int chain = 8 * par + l;
    const int row0 = blockIdx.x * 8;
    const size_t row_bytes = (size_t)K / 2;
    const int ns = (int)(row_bytes / kStripe);
    unsigned char *ring = lds;
    float *act = (float *)(lds + (size_t)D * SLOT);
    float *red = act + F::row_floats(K);   // [2 waves][64 lanes]

    // Stripe DMA (wave 0): lane t fetches row t/8, chunk (t & 7) ^ ((row >> 1) & 7).
    const int dr = lane >> 3;
    const uint8_t *src = W + (size_t)min(row0 + dr, N - 1) * row_bytes + (((lane & 7) ^ ((dr >> 1) & 7)) << 4);
    auto issue = [&](int st) {
        __builtin_amdgcn_global_load_lds((const void *)(src + (size_t)st * kStripe),
                                         (lds_void *)(ring + (st % D) * SLOT), 16, 0, kNT);
    };
    // Activations -> fp32, chain-major (16-byte loads, four per lane in flight).
    {
        const int nvec = K / 8, nthr = 128;
#pragma unroll 1
        for (int v0 = 0; v0 < nvec; v0 += 4 * nthr) {
            u32x4 buf[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int v = v0 + u * nthr + (int)threadIdx.x;
                if (v < nvec) buf[u] = ((const u32x4 *)A)[v];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int v = v0 + u * nthr + (int)threadIdx.x;
                if (v >= nvec) continue;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t word = buf[u][e >> 1];
                    act[F::perm(v * 8 + e)] = (e & 1) ? bf16_hi(word) : bf16_lo(word);
                }
            }
        }
    }
    if (wave == 0) {
#pragma unroll 1
        for (int t = 0; t < D - R; ++t)
            if (t < ns) issue(t);
    }
    // (the first round's barrier orders the activation writes before any read)

    const int swz = (r >> 1) & 7;
    uint32_t off[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) off[j] = r * kStripe + ((j ^ swz) << 4) + 4 * par;
    const int bit = 4 * l;
    float acc = 0.0f;
    uint32_t xw[2][16];
    f32x4 av[2][4];
    auto load = [&](int st, int b) {
        const unsigned char *slot = ring + (st % D) * SLOT;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            xw[b][2 * j] = *(const uint32_t *)(slot + off[j]);
            xw[b][2 * j + 1] = *(const uint32_t *)(slot + off[j] + 8);
        }
        const f32x4 *ap = (const f32x4 *)(act + (st * 16 + chain) * F::kBlock);
#pragma unroll
        for (int v = 0; v < 4; ++v) av[b][v] = ap[v];
    };
    auto compute = [&](int b) {
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const float w = (float)(int)__builtin_amdgcn_sbfe((int)xw[b][t], bit, 4);
            acc = __builtin_fmaf(av[b][t >> 2][t & 3], w, acc);
        }
    };
    const int nfull = ns / R * R;
#pragma unroll 1
    for (int s0 = 0; s0 < nfull; s0 += R) {
        if (wave == 0) {
            if (s0 + D - R - 1 < ns)
                wait_vmcnt<D - 2 * R>();   // stripes s0+R .. s0+D-R-1 may still fly
            else
                wait_vmcnt<0>();
        }
        lds_sync();
        if (wave == 0) {
#pragma unroll
            for (int u = 0; u < R; ++u)
                if (s0 + D - R + u < ns) issue(s0 + D - R + u);
        }
        load(s0, 0);
#pragma unroll
        for (int u = 0; u < R; ++u) {
            __builtin_amdgcn_sched_barrier(0);
            if (u + 1 < R) load(s0 + u + 1, (u + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
            compute(u & 1);
        }
    }
#pragma unroll 1
    for (int s = nfull; s < ns; ++s) {
        if (wave == 0) wait_vmcnt<0>();
        lds_sync();
        load(s, 0);
        compute(0);
    }

    red[wave * 64 + lane] = acc;
    lds_sync();
    const int n = row0 + r;
    if (wave != 0 || c != 0 || n >= N) return;
    float l8[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const float *rw = red + (q >> 2) * 64 + 8 * r + (q & 3);   // wave q/4, lanes c = q & 3 (lo), + 4 (hi)
        l8[q] = rw[0] + rw[4];
    }
    C[n] = f32_to_bf16(hsum8(l8) * S[n]);
}

template <int D>
size_t w4c8_lds_bytes(int K) {
    return (size_t)D * 8 * kStripe + (size_t)(K / 16) * ChainFmt<F_W4ROW, 4>::kBlock * 4 + 2 * 64 * 4;
}

template <int D>
int launch_w4c8(hipStream_t st, const void *A, const uint8_t *W, const float *S, void *C, int N, int K) {
    static std::once_flag once;
    static hipError_t attr_rc = hipSuccess;
    std::call_once(once, [] {
        attr_rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_w4c8_kernel<D>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRowMaxLds);
    });
    if (attr_rc != hipSuccess) return ECPU_ERR_DEVICE;
    const size_t lds = w4c8_lds_bytes<D>(K);
    if (lds > kRowMaxLds) return ECPU_ERR_UNSUPPORTED;
    gemv_w4c8_kernel<D><<<(unsigned)((N + 7) / 8), 128, lds, st>>>((const uint16_t *)A, W, S, (uint16_t *)C, N, K);
    return ECPU_OK;
}

// ------------------------------------------------------------------ byte waves
// W8A32 / W8A16 decode (M = 1), a few thousand rows: the chain kernel pays
// three VALU instructions per weight because a lane's byte position inside
// a dword differs from lane to lane (bit-field extract + conversion + FMA).
// Here a tile of ROWS = 16 or 32 rows has four waves and wave b owns byte b
// of every dword: the eight chains k = 8T + 4p + b of a row are (parity p,
// byte b), so each lane (row r = 16h + t, parity p: DPP row j = p + 2h,
// t = lane & 15; with 16-row tiles DPP rows 2, 3 repeat rows 0..15) decodes
// with one v_cvt_f32_i32 whose SDWA operand selects byte b (a compile-time
// byte: one code path per wave), and the activation of step t of the
// stripe, a[128s + 8t + 4p + b], sits in lane t of the DPP row and reaches
// all sixteen rows through row_newbcast inside the FMA.  Two VALU
// instructions per weight, one chain per lane.  16-row tiles spread a few
// thousand rows over every CU (a CU streams only ~25-30 GB/s).  The four
// waves share a ring of D slots (the tile's rows x 128 B of a stripe plus
// its activations), in rounds of four stripes per barrier; the chain
// sums meet in LDS and one lane per row adds them in the reference's order.

// acc = fma(a of lane t of this 16-lane row, w[t], acc) for t = 0..15 in
// order: one chain's sixteen steps of a stripe.  The s_nop covers the two
// wait states a DPP source needs after a VALU write.
__device__ __forceinline__ void w8b_chain16(float &acc, float a, const float (&w)[16]) {
#define PILM_W8B(T, OP) "v_fmac_f32_dpp %0, %1, %" #OP " row_newbcast:" #T " row_mask:0xf bank_mask:0xf\n\t"
    asm volatile("s_nop 1\n\t" PILM_W8B(0, 2) PILM_W8B(1, 3) PILM_W8B(2, 4) PILM_W8B(3, 5) PILM_W8B(4, 6)
                     PILM_W8B(5, 7) PILM_W8B(6, 8) PILM_W8B(7, 9) PILM_W8B(8, 10) PILM_W8B(9, 11) PILM_W8B(10, 12)
                         PILM_W8B(11, 13) PILM_W8B(12, 14) PILM_W8B(13, 15) PILM_W8B(14, 16) PILM_W8B(15, 17)
                 : "+v"(acc)
                 : "v"(a), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]),
                   "v"(w[8]), "v"(w[9]), "v"(w[10]), "v"(w[11]), "v"(w[12]), "v"(w[13]), "v"(w[14]), "v"(w[15]));
#undef PILM_W8B
}

template <int FMT, int ROWS>
struct W8bFmt {
    static constexpr int ES = FMT == F_W8A32 ? 4 : 2;   // activation bytes
    static constexpr int RB = 128 * ES;                  // activation bytes per stripe
    static constexpr int WB = ROWS * kStripe;            // weight bytes per stripe
    static constexpr int SLOT = WB + RB;                 // the rows' stripe, then the activations
};

template <int FMT, int D, int ROWS>
__global__ __launch_bounds__(256) void gemv_w8b_kernel(const void *__restrict__ A_, const uint8_t *__restrict__ W,
                                                      const float *__restrict__ S, void *__restrict__ C, int N,
                                                      int K) {
    using B8 = W8bFmt<FMT, ROWS>;
    static_assert(ROWS == 8 || ROWS == 16 || ROWS == 32, "tile height");
    constexpr int R = 4;   // stripes per round
    static_assert(D % R == 0 && D >= 2 * R, "ring depth");
    extern __shared__ __align__(16) unsigned char lds[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    // (8-row tiles: lanes t >= 8 repeat rows t - 8, each DPP row still
    // carrying the stripe's sixteen steps)
    const int t = lane & 15, j = lane >> 4, p = j & 1;
    const int r = ROWS == 32 ? 16 * (j >> 1) + t : (ROWS == 16 ? t : (t & 7));
    const int row0 = blockIdx.x * ROWS;
    const int ns = K / kStripe;
    const unsigned char *A = (const unsigned char *)A_;

    // DMA: wave w < ROWS/8 fetches rows 8w + lane/8 of the tile, chunk
    // (lane & 7) ^ ((row >> 1) & 7); the stripe's activations are fetched by
    // the first RB/16 lanes of wave 0.
    constexpr int kIssuers = ROWS / 8;
    const int dr = 8 * (wave % kIssuers) + (lane >> 3);
    const uint8_t *wsrc = W + (size_t)min(row0 + dr, N - 1) * K + (((lane & 7) ^ ((dr >> 1) & 7)) << 4);
    const unsigned char *asrc = A + 16 * lane;
    const bool act_lane = wave == 0 && lane < B8::RB / 16;
    auto issue = [&](int st) {
        unsigned char *slot = lds + (st % D) * B8::SLOT;
        if (wave < kIssuers)
            __builtin_amdgcn_global_load_lds((const void *)(wsrc + (size_t)st * kStripe),
                                             (lds_void *)(slot + wave * 1024), 16, 0, kNT);
        if (wave == 0) {
            if (act_lane)
                __builtin_amdgcn_global_load_lds((const void *)(asrc + (size_t)st * B8::RB),
                                                 (lds_void *)(slot + B8::WB), 16, 0, 0);
        }
    };
#pragma unroll 1
    for (int st = 0; st < D - R && st < ns; ++st) issue(st);

    const int swz = (r >> 1) & 7;
    uint32_t off[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) off[jj] = r * kStripe + ((jj ^ swz) << 4) + 4 * p;
    float acc = 0.0f;

    auto run = [&](auto bc) {
        constexpr int BYTE = decltype(bc)::value;
        // DMA instructions this wave issues per stripe: wave 0 two, the other
        // issuers one, the rest none
        constexpr int PERW = BYTE == 0 ? 2 : (BYTE < kIssuers ? 1 : 0);
        const int aoff = B8::WB + (8 * t + 4 * p + BYTE) * B8::ES;
        uint32_t xw[2][16];
        float av[2];
        auto load = [&](int st, int b) {
            const unsigned char *slot = lds + (st % D) * B8::SLOT;
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                xw[b][2 * jj] = *(const uint32_t *)(slot + off[jj]);
                xw[b][2 * jj + 1] = *(const uint32_t *)(slot + off[jj] + 8);
            }
            if constexpr (FMT == F_W8A32)
                av[b] = *(const float *)(slot + aoff);
            else
                av[b] = __uint_as_float((uint32_t)(*(const uint16_t *)(slot + aoff)) << 16);
        };
        auto compute = [&](int b) {
            float w[16];
#pragma unroll
            for (int q = 0; q < 16; ++q) w[q] = (float)(int)(int8_t)(uint8_t)(xw[b][q] >> (8 * BYTE));
            w8b_chain16(acc, av[b], w);
        };
        const int nfull = ns / R * R;
#pragma unroll 1
        for (int s0 = 0; s0 < nfull; s0 += R) {
            if (s0 + D - R - 1 < ns)
                wait_vmcnt<PERW *(D - 2 * R)>();   // stripes s0+R .. s0+D-R-1 may still fly
            else
                wait_vmcnt<0>();
            lds_sync();
#pragma unroll
            for (int u = 0; u < R; ++u)
                if (s0 + D - R + u < ns) issue(s0 + D - R + u);
            load(s0, 0);
#pragma unroll
            for (int u = 0; u < R; ++u) {
                __builtin_amdgcn_sched_barrier(0);
                if (u + 1 < R) load(s0 + u + 1, (u + 1) & 1);
                __builtin_amdgcn_sched_barrier(0);
                compute(u & 1);
            }
        }
#pragma unroll 1
        for (int s = nfull; s < ns; ++s) {
            wait_vmcnt<0>();
            lds_sync();
            load(s, 0);
            compute(0);
        }
    };
    switch (wave) {
        case 0: run(std::integral_constant<int, 0>{}); break;
        case 1: run(std::integral_constant<int, 1>{}); break;
        case 2: run(std::integral_constant<int, 2>{}); break;
        default: run(std::integral_constant<int, 3>{}); break;
    }

    // red[row][chain l = 4p + b] (16-row tiles: DPP rows 2, 3 store the same
    // values as rows 0, 1; 8-row tiles: lanes t >= 8 the same as t - 8); lane
    // r of wave 0 adds row r's chains.
    float *red = (float *)lds;
    lds_sync();
    red[r * 8 + 4 * p + wave] = acc;
    lds_sync();
    const int n = row0 + lane;
    if (wave != 0 || lane >= ROWS || n >= N) return;
    float l8[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) l8[l] = red[lane * 8 + l];
    const float y = hsum8(l8) * S[n];
    if constexpr (FMT == F_W8A32)
        ((float *)C)[n] = y;
    else
        ((uint16_t *)C)[n] = f32_to_bf16(y);
}

template <int FMT, int ROWS, int D>
int launch_w8b_one(hipStream_t st, const void *A, const uint8_t *W, const float *S, void *C, int N, int K) {
    constexpr size_t lds = (size_t)D * W8bFmt<FMT, ROWS>::SLOT;
    static_assert(lds <= kRowMaxLds, "byte-wave ring");
    static std::once_flag once;
    static hipError_t attr_rc = hipSuccess;
    std::call_once(once, [] {
        attr_rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_w8b_kernel<FMT, D, ROWS>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRowMaxLds);
    });
    if (attr_rc != hipSuccess) return ECPU_ERR_DEVICE;
    gemv_w8b_kernel<FMT, D, ROWS><<<(unsigned)((N + ROWS - 1) / ROWS), 256, lds, st>>>(A, W, S, C, N, K);
    return ECPU_OK;
}

template <int FMT>
int launch_w8b(hipStream_t st, const void *A, const uint8_t *W, const float *S, void *C, int N, int K) {
    // 8-row tiles up to 1024 rows (k/v: 1024x4096 W8A16 9.6 -> 8.9 us; the
    // repeated lanes cost more than the extra CUs gain beyond), 16 below 8192
    // -- for W8A16 below 4096 only (interleaved same-process A/B, 16 vs 32
    // rows: W8A16 4096x12288 26.9 vs 25.0 us, 4096x4096 10.1 vs 9.8 us;
    // W8A32 23.9 vs 25.5 us, 9.6 vs 10.0 us).
    int rows = N <= 1024 ? 8 : (N < (FMT == F_W8A16 ? 4096 : 8192) ? 16 : 32);
    const int env_rows = env_int("PILM_HIP_W8B_ROWS", 0);
    if (env_rows == 8 || env_rows == 16 || env_rows == 32) rows = env_rows;
    // (a 32-slot ring measured slower at every shape: 4096x4096 11.2 vs 9.8 us)
    if (rows == 8) return launch_w8b_one<FMT, 8, 16>(st, A, W, S, C, N, K);
    return rows == 16 ? launch_w8b_one<FMT, 16, 16>(st, A, W, S, C, N, K)
                      : launch_w8b_one<FMT, 32, 16>(st, A, W, S, C, N, K);
}

// ------------------------------------------------------------------ row broadcast
// Per-row formats with a few activation rows (MTP verify M = 1 + drafts,
// short prefills): each weight feeds M FMAs, so the exact path is bound by
// FMA issue, and reading every activation per lane from LDS (the chain
// kernel) or unpacking bf16 pairs per FMA (the quad kernel) costs as much
// again.  Here the 16-row tile keeps the quad layout's chain groups but
// orders the lanes by group, lane = 16c + r, so each 16-lane DPP row holds
// one chain group for 16 rows and every lane of it meets the same activation
// at each step: lane t of the row holds step t's activation for the stripe,
// and v_fmac_f32_dpp row_newbcast:t hands it to all sixteen inside the FMA
// (the single rounding of fmaf).  CS waves per tile divide the chain slots
// (one chain per lane); each weight is decoded once (bit-field extract +
// conversion) and used by MT activation rows.  The waves share a ring of D
// slots, each holding one stripe of the 16 rows' weights and of the MT
// activation rows (wave 0 issues the DMA, one barrier per stripe); chain sums
// meet in LDS and one lane per row adds them in the reference's order.  The
// m-groups of MT rows are the grid's second dimension.

// Step T of eight chains: acc[j] += a[j] of lane T of this 16-lane row times
// w[j].  The s_nop covers the two wait states a DPP source needs after a VALU
// write (the compiler does not see hazards inside inline asm).
template <int T>
__device__ __forceinline__ void rbc_step8(float (&acc)[8], const float (&a)[8], const float (&w)[8]);
template <int T>
__device__ __forceinline__ void rbc_step4(float (&acc)[4], const float (&a)[4], const float (&w)[4]);
template <int T>
__device__ __forceinline__ void rbc_step5(float (&acc)[5], const float (&a)[5], const float (&w)[5]);

#define PILM_RBC_DPP(T) " row_newbcast:" #T " row_mask:0xf bank_mask:0xf\n\t"
#define PILM_RBC_DEF(T)                                                                                           \
    template <>                                                                                                   \
    __device__ __forceinline__ void rbc_step8<T>(float (&acc)[8], const float (&a)[8], const float (&w)[8]) {      \
        asm volatile("s_nop 1\n\t"                                                                                \
                     "v_fmac_f32_dpp %0, %8, %16" PILM_RBC_DPP(T) "v_fmac_f32_dpp %1, %9, %17" PILM_RBC_DPP(T)    \
                     "v_fmac_f32_dpp %2, %10, %18" PILM_RBC_DPP(T) "v_fmac_f32_dpp %3, %11, %19" PILM_RBC_DPP(T)  \
                     "v_fmac_f32_dpp %4, %12, %20" PILM_RBC_DPP(T) "v_fmac_f32_dpp %5, %13, %21" PILM_RBC_DPP(T)  \
                     "v_fmac_f32_dpp %6, %14, %22" PILM_RBC_DPP(T) "v_fmac_f32_dpp %7, %15, %23" PILM_RBC_DPP(T)  \
                     : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), "+v"(acc[4]), "+v"(acc[5]),       \
                       "+v"(acc[6]), "+v"(acc[7])                                                                 \
                     : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]),    \
                       "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]));   \
    }                                                                                                             \
    template <>                                                                                                   \
    __device__ __forceinline__ void rbc_step4<T>(float (&acc)[4], const float (&a)[4], const float (&w)[4]) {      \
        asm volatile("s_nop 1\n\t"                                                                                \
                     "v_fmac_f32_dpp %0, %4, %8" PILM_RBC_DPP(T) "v_fmac_f32_dpp %1, %5, %9" PILM_RBC_DPP(T)      \
                     "v_fmac_f32_dpp %2, %6, %10" PILM_RBC_DPP(T) "v_fmac_f32_dpp %3, %7, %11" PILM_RBC_DPP(T)    \
                     : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3])                                     \
                     : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]));   \
    }                                                                                                             \
    template <>                                                                                                   \
    __device__ __forceinline__ void rbc_step5<T>(float (&acc)[5], const float (&a)[5], const float (&w)[5]) {      \
        asm volatile("s_nop 1\n\t"                                                                                \
                     "v_fmac_f32_dpp %0, %5, %10" PILM_RBC_DPP(T) "v_fmac_f32_dpp %1, %6, %11" PILM_RBC_DPP(T)    \
                     "v_fmac_f32_dpp %2, %7, %12" PILM_RBC_DPP(T) "v_fmac_f32_dpp %3, %8, %13" PILM_RBC_DPP(T)    \
                     "v_fmac_f32_dpp %4, %9, %14" PILM_RBC_DPP(T)                                                 \
                     : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), "+v"(acc[4])                       \
                     : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(w[0]), "v"(w[1]), "v"(w[2]),    \
                       "v"(w[3]), "v"(w[4]));                                                                     \
    }
PILM_RBC_DEF(0) PILM_RBC_DEF(1) PILM_RBC_DEF(2) PILM_RBC_DEF(3) PILM_RBC_DEF(4) PILM_RBC_DEF(5) PILM_RBC_DEF(6)
PILM_RBC_DEF(7) PILM_RBC_DEF(8) PILM_RBC_DEF(9) PILM_RBC_DEF(10) PILM_RBC_DEF(11) PILM_RBC_DEF(12)
PILM_RBC_DEF(13) PILM_RBC_DEF(14) PILM_RBC_DEF(15)
#undef PILM_RBC_DEF
#undef PILM_RBC_DPP

template <int FMT, int MT, int CS>
struct RbcFmt {
    using F = ChainFmt<FMT, CS>;
    static constexpr int SL = F::slots;                        // chains per lane
    static constexpr int NF = MT * SL;                         // FMAs per lane and step (4, 5 or 8)
    static_assert(NF == 4 || NF == 5 || NF == 8, "row-broadcast step width");
    static constexpr int ES = FMT == F_W8A32 ? 4 : 2;          // activation bytes
    static constexpr int SPE = F::w8 ? 128 : 256;              // row elements per stripe
    static constexpr int STEP = F::w8 ? 8 : 16;                // elements per step (a chain takes one)
    static constexpr int RB = SPE * ES;                        // activation bytes of a row per stripe
    // activation bytes per slot, in whole 1 KB DMA instructions (five rows:
    // the padding repeats the last row and is not read)
    static constexpr int ACT = (MT * RB + 1023) / 1024 * 1024;
    static constexpr int SLOT = kQuadSlotBytes + ACT;          // weights (16 rows x 128 B) + activations
    static constexpr int PER = 2 + ACT / 1024;                 // DMA instructions per stripe
};

template <int FMT, int MT, int CS, int D>
__global__ __launch_bounds__(64 * CS) void gemv_rbc_kernel(const void *__restrict__ A_, const uint8_t *__restrict__ W,
                                                          const float *__restrict__ S, void *__restrict__ C, int M,
                                                          int N, int K) {
    using R = RbcFmt<FMT, MT, CS>;
    using F = typename R::F;
    constexpr int SL = R::SL;
    static_assert(R::PER * (D - 2) < 64, "vmcnt range");
    extern __shared__ __align__(16) unsigned char lds[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int r = lane & 15, c = lane >> 4, par = c >> 1, t16 = lane & 15;
    const int row0 = blockIdx.x * 16;
    const int mb = (int)blockIdx.y * MT;
    const int mvalid = min(MT, M - mb);
    const size_t row_bytes = F::w8 ? (size_t)K : (size_t)K / 2;
    const int ns = (int)(row_bytes / kStripe);
    const unsigned char *A = (const unsigned char *)A_;

    // DMA (wave 0): instructions 0, 1 fetch rows 8i + lane/8 of the tile,
    // chunk (lane & 7) ^ ((row >> 1) & 7); instructions 2.. fetch 1 KB of the
    // stripe's activation rows each (rows past M repeat the last row).
    const uint8_t *wsrc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int rr = 8 * i + (lane >> 3);
        wsrc[i] = W + (size_t)min(row0 + rr, N - 1) * row_bytes + (((lane & 7) ^ ((rr >> 1) & 7)) << 4);
    }
    const unsigned char *asrc[R::PER - 2];
#pragma unroll
    for (int j = 0; j < R::PER - 2; ++j) {
        const int b = j * 1024 + 16 * lane;
        const int m = b / R::RB;
        asrc[j] = A + ((size_t)(mb + min(m, mvalid - 1)) * K) * R::ES + (b - m * R::RB);
    }
    auto issue = [&](int st) {
        unsigned char *slot = lds + (st % D) * R::SLOT;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(wsrc[i] + (size_t)st * kStripe),
                                             (lds_void *)(slot + i * 1024), 16, 0, kNT);
#pragma unroll
        for (int j = 0; j < R::PER - 2; ++j)
            __builtin_amdgcn_global_load_lds((const void *)(asrc[j] + (size_t)st * R::RB),
                                             (lds_void *)(slot + kQuadSlotBytes + j * 1024), 16, 0, 0);
    };
    if (wave == 0) {
#pragma unroll 1
        for (int st = 0; st < D - 1 && st < ns; ++st) issue(st);
    }

    const int swz = (r >> 1) & 7;
    uint32_t off[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) off[j] = r * kStripe + ((j ^ swz) << 4) + 4 * par;
    int bits[SL], aoff[SL];
#pragma unroll
    for (int i = 0; i < SL; ++i) {
        bits[i] = F::bit(c, wave * SL + i);
        aoff[i] = (R::STEP * t16 + F::chain(c, wave * SL + i)) * R::ES;   // lane t16 holds step t16's value
    }
    float acc[MT][SL];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int i = 0; i < SL; ++i) acc[m][i] = 0.0f;

#pragma unroll 1
    for (int s = 0; s < ns; ++s) {
        if (wave == 0) {
            if (s + D - 2 < ns)
                wait_vmcnt<R::PER * (D - 2)>();   // stripes s+1 .. s+D-2 may still fly
            else
                wait_vmcnt<0>();
        }
        // stripe s landed for everyone; every wave is done with slot (s-1) % D
        asm volatile("s_barrier" ::: "memory");
        if (wave == 0 && s + D - 1 < ns) issue(s + D - 1);
        const unsigned char *slot = lds + (s % D) * R::SLOT;
        uint32_t x[16];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            x[2 * j] = *(const uint32_t *)(slot + off[j]);
            x[2 * j + 1] = *(const uint32_t *)(slot + off[j] + 8);
        }
        float av[R::NF];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int i = 0; i < SL; ++i) {
                const unsigned char *ap = slot + kQuadSlotBytes + m * R::RB + aoff[i];
                if constexpr (FMT == F_W8A32)
                    av[m * SL + i] = *(const float *)ap;
                else
                    av[m * SL + i] = __uint_as_float((uint32_t)(*(const uint16_t *)ap) << 16);
            }
        float fa[R::NF];
#pragma unroll
        for (int q = 0; q < R::NF; ++q) fa[q] = acc[q / SL][q % SL];
        auto step = [&](auto tc) {
            constexpr int T = decltype(tc)::value;
            float w[R::NF];
#pragma unroll
            for (int i = 0; i < SL; ++i) {
                const float wi = (float)(int)__builtin_amdgcn_sbfe((int)x[T], bits[i], F::width);
#pragma unroll
                for (int m = 0; m < MT; ++m) w[m * SL + i] = wi;
            }
            if constexpr (R::NF == 8)
                rbc_step8<T>(fa, av, w);
            else if constexpr (R::NF == 5)
                rbc_step5<T>(fa, av, w);
            else
                rbc_step4<T>(fa, av, w);
        };
        step(std::integral_constant<int, 0>{});
        step(std::integral_constant<int, 1>{});
        step(std::integral_constant<int, 2>{});
        step(std::integral_constant<int, 3>{});
        step(std::integral_constant<int, 4>{});
        step(std::integral_constant<int, 5>{});
        step(std::integral_constant<int, 6>{});
        step(std::integral_constant<int, 7>{});
        step(std::integral_constant<int, 8>{});
        step(std::integral_constant<int, 9>{});
        step(std::integral_constant<int, 10>{});
        step(std::integral_constant<int, 11>{});
        step(std::integral_constant<int, 12>{});
        step(std::integral_constant<int, 13>{});
        step(std::integral_constant<int, 14>{});
        step(std::integral_constant<int, 15>{});
#pragma unroll
        for (int q = 0; q < R::NF; ++q) acc[q / SL][q % SL] = fa[q];
    }

    // Chain sums meet in LDS (over the ring, once every wave is done with it):
    // red[m][gslot][c][r]; lane r < 16 of wave 0 adds row r's chains in the
    // reference's order: hsum ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)) of the 8
    // lanes (int4: of lo[l] + hi[l]), times the row scale.
    float *red = (float *)lds;
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int i = 0; i < SL; ++i) red[((m * F::gslots + wave * SL + i) * 4 + c) * 16 + r] = acc[m][i];
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const int n = row0 + lane;
    if (wave != 0 || lane >= 16 || n >= N) return;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        if (m >= mvalid) break;
        const float *rm = red + m * F::gslots * 64 + lane;   // [gslot][c] at (g * 4 + c) * 16
        float l8[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            if constexpr (F::w8) {
                const int g = l & 1, cc = 2 * (l >> 2) + ((l >> 1) & 1);
                l8[l] = rm[(g * 4 + cc) * 16];
            } else {
                const int g = ((l >> 2) & 1) + 2 * (l & 1), cl = (l >> 1) & 1;
                l8[l] = rm[(g * 4 + cl) * 16] + rm[(g * 4 + cl + 2) * 16];
            }
        }
        const float y = hsum8(l8) * S[n];
        const size_t o = (size_t)(mb + m) * N + n;
        if constexpr (FMT == F_W8A32)
            ((float *)C)[o] = y;
        else
            ((uint16_t *)C)[o] = f32_to_bf16(y);
    }
}

template <int FMT, int MT, int CS, int D>
constexpr size_t rbc_lds_bytes() {
    using R = RbcFmt<FMT, MT, CS>;
    const size_t ring = (size_t)D * R::SLOT, red = (size_t)MT * R::F::gslots * 64 * sizeof(float);
    return ring > red ? ring : red;
}

template <int FMT, int MT, int CS>
int launch_rbc_one(int ntiles, int mgroups, hipStream_t st, const void *A, const uint8_t *W, const float *S, void *C,
                   int M, int N, int K) {
    constexpr int D = 8;
    constexpr size_t lds = rbc_lds_bytes<FMT, MT, CS, D>();
    static_assert(lds <= kRowMaxLds, "row-broadcast ring");
    static std::once_flag once;
    static hipError_t attr_rc = hipSuccess;
    std::call_once(once, [] {
        attr_rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_rbc_kernel<FMT, MT, CS, D>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRowMaxLds);
    });
    if (attr_rc != hipSuccess) return ECPU_ERR_DEVICE;
    gemv_rbc_kernel<FMT, MT, CS, D><<<dim3((unsigned)ntiles, (unsigned)mgroups), 64 * CS, lds, st>>>(A, W, S, C, M, N,
                                                                                                     K);
    return ECPU_OK;
}

// Per-row formats, 3 <= M < 64: one chain per lane (W8 over two waves per
// tile, W4 over four), MT = 8 activation rows per wave where that computes
// no more padding rows than MT = 4 and still leaves >= 2048 waves, MT = 5
// for five rows on larger shapes (below), else 4
// (measured: W8A16 8192x4096 M=5 23.1 vs 29.0 us, W4 12288x2048 M=16 25.2
// vs 27.2 us, W4 12288x2048 M=4 10.0 vs 13.5 us).
int run_rbc(int fmt, size_t M, size_t N, size_t K, const void *A, const uint8_t *W, const float *S, void *C,
            hipStream_t st, const char *fn) {
    const int ntiles = (int)((N + 15) / 16);
    const int cs = fmt == F_W4ROW ? 4 : 2;
    const size_t pad8 = (M + 7) / 8 * 8, pad4 = (M + 3) / 4 * 4;
    int mt = pad8 <= pad4 && (size_t)ntiles * cs * (pad8 / 8) >= 2048 ? 8 : 4;
    // MTP verify with four drafts: five rows, no padding, where the tiles
    // alone give enough waves (>= 512 for W8, >= 1024 for W4; below, two
    // m-groups of four spread further): W8A16 24576x4096 51.4 vs 67.5 us,
    // 8192x4096 22.2 vs 23.6 us; 1024x4096 stays at 15.7 (vs 17.3) us.
    if (M == 5 && (size_t)ntiles * cs >= (cs == 4 ? 1024u : 512u))
        mt = 5;
    const int env_mt = env_int("PILM_HIP_RBC_MT", 0);
    if (env_mt == 4 || env_mt == 5 || env_mt == 8) mt = env_mt;
    const size_t mgroups = (M + mt - 1) / mt;
    if (mgroups > 65535) return ECPU_ERR_UNSUPPORTED;
    const int mg = (int)mgroups;
    int rc;
    switch (fmt) {
        case F_W8A32:
            rc = mt == 8   ? launch_rbc_one<F_W8A32, 8, 2>(ntiles, mg, st, A, W, S, C, (int)M, (int)N, (int)K)
                 : mt == 5 ? launch_rbc_one<F_W8A32, 5, 2>(ntiles, mg, st, A, W, S, C, (int)M, (int)N, (int)K)
                           : launch_rbc_one<F_W8A32, 4, 2>(ntiles, mg, st, A, W, S, C, (int)M, (int)N, (int)K);
            break;
        case F_W8A16:
            rc = mt == 8   ? launch_rbc_one<F_W8A16, 8, 2>(ntiles, mg, st, A, W, S, C, (int)M, (int)N, (int)K)
                 : mt == 5 ? launch_rbc_one<F_W8A16, 5, 2>(ntiles, mg, st, A, W, S, C, (int)M, (int)N, (int)K)
                           : launch_rbc_one<F_W8A16, 4, 2>(ntiles, mg, st, A, W, S, C, (int)M, (int)N, (int)K);
            break;
        default:
            rc = mt == 8   ? launch_rbc_one<F_W4ROW, 8, 4>(ntiles, mg, st, A, W, S, C, (int)M, (int)N, (int)K)
                 : mt == 5 ? launch_rbc_one<F_W4ROW, 5, 4>(ntiles, mg, st, A, W, S, C, (int)M, (int)N, (int)K)
                           : launch_rbc_one<F_W4ROW, 4, 4>(ntiles, mg, st, A, W, S, C, (int)M, (int)N, (int)K);
    }
    if (rc != ECPU_OK) return fail(ECPU_ERR_DEVICE, "%s: raising the LDS limit of the small-M kernel failed", fn);
    return ECPU_OK;
}

// ------------------------------------------------------------------ group quad
// Group formats (W4A16 g128 / g32) with the quad layout: 16-row tiles, lane
// 4r + c serves row r with the quad kernel's int4 chains (the packing is the
// per-row format's), and the P waves of a workgroup take consecutive ranges
// of the tile's stripes.  A group's block sum is the int4 dot over the group
// (kernels.c:1130-1140: lo/hi chains over its 16-element chunks, hsum of
// lo + hi), reduced across the quad with DPP in the reference's order as soon
// as the group's words are done; lane c = 0 parks it in LDS.  After a barrier
// wave 0 folds every row's blocks in group order, acc = fma(block, scale,
// acc), the reference's sequence exactly, so K can be divided among the
// waves without changing a bit.  The row scales of the tile are copied to
// LDS at the start (DMA, behind the activations), so the fold waits for
// nothing.
// Optional GemmaRMSNorm prologue of the group-quad kernel (one activation
// row): h = bf16(x + res) (or x), res_out = h (workgroup 0), and the
// activation row a = bf16(bf16(w + 1) * bf16(h * r)), r = 1 / sqrt(mean(h^2)
// + eps) in torch's CPU order, computed by every workgroup into its LDS copy
// of the activations.
struct GqNorm {
    const uint16_t *x = nullptr;
    const uint16_t *res = nullptr;
    const uint16_t *w = nullptr;
    uint16_t *res_out = nullptr;
    float eps = 0.0f;
};
constexpr int kGqNormChunks = 4;   // eight-element chunks of the row per thread

template <int FMT, int MT, int D, int P, bool NORM = false, bool SW = false>
__global__ __launch_bounds__(64 * P) void gemv_gq_kernel(const uint16_t *__restrict__ A, const uint8_t *__restrict__ W,
                                                     const float *__restrict__ S, uint16_t *__restrict__ C, int N,
                                                     int K, int m0, GqNorm na) {
    using Q = QuadFmt<F_W4ROW>;
    static_assert(!(NORM || SW) || MT == 1, "norm prologue / SwiGLU epilogue: one activation row");
    constexpr int GS = FMT == F_W4G128 ? 128 : 32;   // group size
    constexpr int GPS = 256 / GS;                    // groups per stripe: 2 or 8
    constexpr int WPG = 16 / GPS;                    // lane words per group: 8 or 2
    extern __shared__ __align__(16) unsigned char lds[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int r = lane >> 2, c = lane & 3, par = c >> 1;
    const int row0 = blockIdx.x * 16;
    // weight row of tile row rr: SW pairs gate rows 8t..8t+7 (tile rows 0-7)
    // with their up rows N/2 + 8t.. (tile rows 8-15)
    auto wrow = [&](int rr) -> size_t {
        if constexpr (SW)
            return rr < 8 ? (size_t)blockIdx.x * 8 + rr : (size_t)(N / 2) + blockIdx.x * 8 + (rr - 8);
        else
            return (size_t)min(row0 + rr, N - 1);
    };
    const size_t row_bytes = (size_t)K / 2;
    const int ns = (int)(row_bytes / kStripe);
    const int G = K / GS;
    const int rdw = K / 2;                          // activation dwords per row
    const int sps = (ns + P - 1) / P;
    const int sb = min(ns, wave * sps);
    const int nsw = min(ns, sb + sps) - sb;         // this wave's stripes (may be 0)
    unsigned char *act = lds + (size_t)P * D * kQuadSlotBytes;
    float *scl = (float *)(act + (size_t)MT * rdw * 4);   // [16][G]
    float *blk = scl + 16 * G;                             // [MT][16][G]

    // Activation rows (16-byte DMA, 256 dwords per instruction; NORM: computed
    // below instead) and the tile's scales (4-byte DMA, 64 per instruction),
    // dealt round-robin.
    {
        int issued = 0;
        if constexpr (!NORM) {
            const int total = MT * rdw;
            const uint32_t *a = (const uint32_t *)A + (size_t)m0 * rdw;
#pragma unroll 1
            for (int q = wave; q * 256 < total; q += P) {
                const int g = q * 256 + 4 * lane;
                if (g < total)
                    __builtin_amdgcn_global_load_lds((const void *)(a + g), (lds_void *)(act + (size_t)q * 1024), 16,
                                                     0, 0);
                if ((++issued & 15) == 0) wait_vmcnt<16>();
            }
        }
        const int nscl = 16 * G;
#pragma unroll 1
        for (int q = wave; q * 64 < nscl; q += P) {
            const int i = q * 64 + lane;
            if (i < nscl) {
                const int rr = i / G, g = i - rr * G;
                __builtin_amdgcn_global_load_lds((const void *)(S + wrow(rr) * G + g), (lds_void *)(scl + q * 64), 4,
                                                 0, 0);
            }
            if ((++issued & 15) == 0) wait_vmcnt<16>();
        }
    }

    // This wave's stripes sb .. sb+nsw-1 through its own ring of D slots.
    const uint8_t *src[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int rr = 8 * i + (lane >> 3);
        const int q = (lane & 7) ^ ((rr >> 1) & 7);
        src[i] = W + wrow(rr) * row_bytes + q * 16;
    }
    unsigned char *ring = lds + (size_t)wave * D * kQuadSlotBytes;
    auto issue = [&](int t) {   // t: index within this wave's range
        unsigned char *slot = ring + (t % D) * kQuadSlotBytes;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(src[i] + (size_t)(sb + t) * kStripe),
                                             (lds_void *)(slot + i * 1024), 16, 0, kNT);
    };
#pragma unroll
    for (int t = 0; t < D - 2; ++t)
        if (t < nsw) issue(t);
    if constexpr (NORM) {
        // the row, its residual and the norm weight in 16-byte chunks (the
        // first stripes are already on their way), then the norm into act
        float *xs = blk + 16 * G;                  // [K + 4]: h as fp32, then r
        const int nc = K / 8, t = threadIdx.x;
        u32x4 xv[kGqNormChunks], rv[kGqNormChunks], wv[kGqNormChunks];
#pragma unroll
        for (int u = 0; u < kGqNormChunks; ++u) {
            const int ch = t + 64 * P * u;
            if (ch < nc) {
                xv[u] = ((const u32x4 *)na.x)[ch];
                if (na.res) rv[u] = ((const u32x4 *)na.res)[ch];
                wv[u] = ((const u32x4 *)na.w)[ch];
            }
        }
        float h[kGqNormChunks][8];
#pragma unroll
        for (int u = 0; u < kGqNormChunks; ++u) {
            const int ch = t + 64 * P * u;
            if (ch < nc) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float lo = bf16_lo(xv[u][e]), hi = bf16_hi(xv[u][e]);
                    if (na.res) {
                        lo = bfr(lo + bf16_lo(rv[u][e]));
                        hi = bfr(hi + bf16_hi(rv[u][e]));
                    }
                    h[u][2 * e] = lo;
                    h[u][2 * e + 1] = hi;
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) xs[8 * ch + e] = h[u][e];
                if (na.res_out && blockIdx.x == 0) {
                    u32x4 o;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        o[e] = (uint32_t)f32_to_bf16(h[u][2 * e]) | ((uint32_t)f32_to_bf16(h[u][2 * e + 1]) << 16);
                    ((u32x4 *)na.res_out)[ch] = o;
                }
            }
        }
        __syncthreads();
        // torch's sum of squares: its 16-vector block sums by every thread,
        // then one wave replays the cascade and the fold
        float *bs = xs + K + 4;                    // [32 (K / 512 + 1)]
        row_sumsq_blocks(xs, K, bs, threadIdx.x, 64 * P);
        __syncthreads();
        if (wave == 0) {
            const float rs = wave_row_rsqrt_blocks(xs, bs, K, na.eps);
            if (lane == 0) xs[K] = rs;
        }
        __syncthreads();
        const float rs = xs[K];
#pragma unroll
        for (int u = 0; u < kGqNormChunks; ++u) {
            const int ch = t + 64 * P * u;
            if (ch < nc) {
                u32x4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    o[e] = (uint32_t)gemma_out(h[u][2 * e], rs, (uint16_t)(wv[u][e] & 0xFFFFu)) |
                           ((uint32_t)gemma_out(h[u][2 * e + 1], rs, (uint16_t)(wv[u][e] >> 16)) << 16);
                ((u32x4 *)act)[ch] = o;
            }
        }
        __syncthreads();                           // the activation row is in
    }
    if (nsw >= D - 2)
        wait_vmcnt<2 * (D - 2)>();   // activation and scale copies, older than the stripes
    else
        wait_vmcnt<0>();
    asm volatile("s_barrier" ::: "memory");

    const int swz = (r >> 1) & 7;
    uint32_t off[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) off[j] = r * kStripe + ((j ^ swz) << 4) + 4 * par;
    const uint32_t *my_act = (const uint32_t *)act + Q::act_index(0, c);
    const uint32_t shift = 8u * (c & 1);
    const uint32_t magic = opaque_magic();

    float acc[MT][4];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[m][k] = 0.0f;

    auto load = [&](int t, uint32_t (&x)[16], uint32_t (&av)[MT][32]) {
        const unsigned char *slot = ring + (t % D) * kQuadSlotBytes;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            x[2 * j] = *(const uint32_t *)(slot + off[j]);
            x[2 * j + 1] = *(const uint32_t *)(slot + off[j] + 8);
        }
        const int st = sb + t;
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const uint32_t *ap = my_act + (size_t)m * rdw + Q::act_index(16 * st + u, 0);
                av[m][2 * u] = ap[0];
                av[m][2 * u + 1] = ap[2];
            }
    };
    // One stripe: GPS groups of WPG words each; after each group its block
    // sums are reduced across the quad and parked.
    auto compute = [&](int t, const uint32_t (&x)[16], const uint32_t (&av)[MT][32]) {
        const int g0 = (sb + t) * GPS;
#pragma unroll
        for (int gi = 0; gi < GPS; ++gi) {
#pragma unroll
            for (int u = gi * WPG; u < (gi + 1) * WPG; ++u) {
                const uint32_t v = (x[u] ^ 0x88888888u) >> shift;
                const h2 bias = {(_Float16)-1032.0f, (_Float16)-1032.0f};
                const h2 sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
                const h2 bias16 = {(_Float16)-72.0f, (_Float16)-72.0f};
                const h2 qa = __builtin_bit_cast(h2, (v & 0x000F000Fu) | magic) + bias;
                const h2 qb = __builtin_bit_cast(h2, (v & 0x00F000F0u) | magic) * sixteenth + bias16;
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const uint32_t p0 = av[m][2 * u], p1 = av[m][2 * u + 1];
                    acc[m][0] = __builtin_fmaf(bf16_lo(p0), (float)qa.x, acc[m][0]);
                    acc[m][1] = __builtin_fmaf(bf16_lo(p1), (float)qa.y, acc[m][1]);
                    acc[m][2] = __builtin_fmaf(bf16_hi(p0), (float)qb.x, acc[m][2]);
                    acc[m][3] = __builtin_fmaf(bf16_hi(p1), (float)qb.y, acc[m][3]);
                }
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float s0 = dpp_quad_add(acc[m][0], 1);
                const float s4 = dpp_quad_add(acc[m][1], 1);
                const float s1 = dpp_quad_add(acc[m][2], 1);
                const float s5 = dpp_quad_add(acc[m][3], 1);
                const float h = dpp_quad_add((s0 + s4) + (s1 + s5), 0);
                if (c == 0) blk[(m * 16 + r) * G + g0 + gi] = h;
#pragma unroll
                for (int k = 0; k < 4; ++k) acc[m][k] = 0.0f;
            }
        }
    };
    uint32_t xa[16], xb[16];
    uint32_t aa[MT][32], ab[MT][32];
    if (nsw > 0) {
        if (nsw >= D - 2)
            wait_vmcnt<2 * (D - 3)>();
        else
            wait_vmcnt<0>();
        load(0, xa, aa);
    }
    int t = 0;
#pragma unroll 1
    for (; t + 1 < nsw; t += 2) {
        if (t + D - 2 < nsw) issue(t + D - 2);
        if (t + D - 1 < nsw) issue(t + D - 1);
        if (t + D <= nsw)
            wait_vmcnt<2 * (D - 2)>();
        else
            wait_vmcnt<0>();
        load(t + 1, xb, ab);
        compute(t, xa, aa);
        if (t + 2 < nsw) {
            if (t + D <= nsw)
                wait_vmcnt<2 * (D - 3)>();
            else
                wait_vmcnt<0>();
            load(t + 2, xa, aa);
        }
        compute(t + 1, xb, ab);
    }
    if (t < nsw) compute(t, xa, aa);

    // Fold: row r's blocks in group order (kernels.c:1141-1150), by lane 4r of wave 0.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if constexpr (SW) {
        // gate row r < 8 and up row r + 8 (lane 4r + 32): C[8t + r] =
        // bf16(bf16(silu(g)) * u), F.silu(gate(x)) * up(x) on the bf16 outputs
        if (wave != 0) return;
        float a = 0.0f;
        if (c == 0) {
            const float *sr = scl + r * G, *br = blk + r * G;
#pragma unroll 8
            for (int g = 0; g < G; ++g) a = __builtin_fmaf(br[g], sr[g], a);
        }
        const float v = bfr(a);
        const float u = __shfl(v, lane + 32);
        if (c == 0 && r < 8) {
            const float sl = bfr(__fdiv_rn(v, 1.0f + sleef_expf(-v)));
            C[(size_t)blockIdx.x * 8 + r] = f32_to_bf16(sl * u);
        }
        return;
    }
    const int n = row0 + r;
    if (wave != 0 || c != 0 || n >= N) return;
    const float *sr = scl + r * G;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const float *br = blk + (m * 16 + r) * G;
        float a = 0.0f;
#pragma unroll 8
        for (int g = 0; g < G; ++g) a = __builtin_fmaf(br[g], sr[g], a);
        C[(size_t)(m0 + m) * N + n] = f32_to_bf16(a);
    }
}

template <int FMT, int MT, int D, int P, bool NORM = false>
size_t gq_lds_bytes(int K) {
    const size_t G = (size_t)K / (FMT == F_W4G128 ? 128 : 32);
    return (size_t)P * D * kQuadSlotBytes + (size_t)MT * K * 2 + 16 * G * 4 + (size_t)MT * 16 * G * 4 +
           (NORM ? ((size_t)K + 4 + 32 * ((size_t)K / 512 + 1)) * 4 : 0);
}

template <int FMT, int MT, int D, int P>
int launch_gq_one(int ntiles, hipStream_t st, const uint16_t *A, const uint8_t *W, const float *S, uint16_t *C,
                  int N, int K, int m0) {
    static std::once_flag once;
    static hipError_t attr_rc = hipSuccess;
    std::call_once(once, [] {
        attr_rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_gq_kernel<FMT, MT, D, P>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRowMaxLds);
    });
    if (attr_rc != hipSuccess) return ECPU_ERR_DEVICE;
    const size_t lds = gq_lds_bytes<FMT, MT, D, P>(K);
    if (lds > kRowMaxLds) return ECPU_ERR_UNSUPPORTED;
    gemv_gq_kernel<FMT, MT, D, P><<<ntiles, 64 * P, lds, st>>>(A, W, S, C, N, K, m0, GqNorm{});
    return ECPU_OK;
}

// One activation row through a GemmaRMSNorm prologue (and with sw, the
// SwiGLU epilogue over gate/up row pairs).
template <bool SW, int P, int D>
static int launch_gq_norm(int ntiles, hipStream_t st, const uint8_t *W, const float *S, uint16_t *C, int N, int K,
                          const GqNorm &na) {
    static std::once_flag once;
    static hipError_t attr_rc = hipSuccess;
    std::call_once(once, [] {
        attr_rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_gq_kernel<F_W4G128, 1, D, P, true, SW>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRowMaxLds);
    });
    if (attr_rc != hipSuccess) return ECPU_ERR_DEVICE;
    const size_t lds = gq_lds_bytes<F_W4G128, 1, D, P, true>(K);
    if (lds > kRowMaxLds) return ECPU_ERR_UNSUPPORTED;
    gemv_gq_kernel<F_W4G128, 1, D, P, true, SW><<<ntiles, 64 * P, lds, st>>>(nullptr, W, S, C, N, K, 0, na);
    return ECPU_OK;
}


template <int FMT, int D, int P>
int launch_gq_mt(int mt, int ntiles, hipStream_t st, const uint16_t *A, const uint8_t *W, const float *S,
                 uint16_t *C, int N, int K, int m0) {
    switch (mt) {
        case 1: return launch_gq_one<FMT, 1, D, P>(ntiles, st, A, W, S, C, N, K, m0);
        case 2: return launch_gq_one<FMT, 2, D, P>(ntiles, st, A, W, S, C, N, K, m0);
        case 3: return launch_gq_one<FMT, 3, D, P>(ntiles, st, A, W, S, C, N, K, m0);
        default: return launch_gq_one<FMT, 4, D, P>(ntiles, st, A, W, S, C, N, K, m0);
    }
}

// 8-row tiles for up to four activation rows (k/v, o, down at 1.7B: 64-128
// 16-row tiles would leave CUs idle, and dividing a tile across workgroups
// costs a global round trip).  Lane 8r + c serves row r: c < 4 the lo half of each
// 16-element chunk, c >= 4 the hi half, chains (c & 3) and (c & 3) + 4 --
// two int4 chains per lane instead of four.  The block sums of a group meet
// in the reference's order: lo + hi (lane c reads lane c + 4 of its 16-lane
// row by DPP row_ror:12), then ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)) by quad
// permutes.
// Otherwise as gemv_gq_kernel (per-wave rings, activations and scales by DMA,
// blocks folded in group order by lane 8r of wave 0).
// Value of lane i + 4 (mod 16) of the 16-lane row: row_ror:12 (lane i reads
// lane i - 12).
__device__ __forceinline__ float dpp_up4(float x) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x12C, 0xF, 0xF, false));
}

template <int FMT, int MT, int D, int P>
__global__ __launch_bounds__(64 * P) void gemv_gq8_kernel(const uint16_t *__restrict__ A, const uint8_t *__restrict__ W,
                                                      const float *__restrict__ S, uint16_t *__restrict__ C, int N,
                                                      int K, int m0) {
    constexpr int GS = FMT == F_W4G128 ? 128 : 32;   // group size
    constexpr int GPS = 256 / GS;                    // groups per stripe: 2 or 8
    constexpr int WPG = 16 / GPS;                    // lane words per group: 8 or 2
    constexpr int SLOT = 8 * kStripe;                // one stripe of the tile: 8 rows x 128 B
    extern __shared__ __align__(16) unsigned char lds[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int r = lane >> 3, c = lane & 7, par = c >> 2, nb = c & 3;
    const int row0 = blockIdx.x * 8;
    const size_t row_bytes = (size_t)K / 2;
    const int ns = (int)(row_bytes / kStripe);
    const int G = K / GS;
    const int rdw = K / 2;                          // activation dwords
    const int sps = (ns + P - 1) / P;
    const int sb = min(ns, wave * sps);
    const int nsw = min(ns, sb + sps) - sb;         // this wave's stripes (may be 0)
    unsigned char *act = lds + (size_t)P * D * SLOT;
    float *scl = (float *)(act + (size_t)MT * rdw * 4);   // [8][G]
    float *blk = scl + 8 * G;                              // [MT][8][G]

    // Activation rows m0.. (16-byte DMA, 256 dwords per instruction) and the
    // tile's scales (4-byte DMA, 64 per instruction), dealt round-robin.
    {
        int issued = 0;
        const int total = MT * rdw;
        const uint32_t *a = (const uint32_t *)A + (size_t)m0 * rdw;
#pragma unroll 1
        for (int q = wave; q * 256 < total; q += P) {
            const int g = q * 256 + 4 * lane;
            if (g < total)
                __builtin_amdgcn_global_load_lds((const void *)(a + g), (lds_void *)(act + (size_t)q * 1024), 16, 0,
                                                 0);
            if ((++issued & 15) == 0) wait_vmcnt<16>();
        }
        const int nscl = 8 * G;
#pragma unroll 1
        for (int q = wave; q * 64 < nscl; q += P) {
            const int i = q * 64 + lane;
            if (i < nscl) {
                const int rr = i / G, g = i - rr * G;
                __builtin_amdgcn_global_load_lds((const void *)(S + (size_t)min(row0 + rr, N - 1) * G + g),
                                                 (lds_void *)(scl + q * 64), 4, 0, 0);
            }
            if ((++issued & 15) == 0) wait_vmcnt<16>();
        }
    }

    // This wave's stripes through its own ring of D slots: lane t fetches
    // row t/8, chunk (t & 7) ^ ((row >> 1) & 7).
    const int rr = lane >> 3;
    const uint8_t *src = W + (size_t)min(row0 + rr, N - 1) * row_bytes + (((lane & 7) ^ ((rr >> 1) & 7)) << 4);
    unsigned char *ring = lds + (size_t)wave * D * SLOT;
    auto issue = [&](int t) {
        __builtin_amdgcn_global_load_lds((const void *)(src + (size_t)(sb + t) * kStripe),
                                         (lds_void *)(ring + (t % D) * SLOT), 16, 0, kNT);
    };
#pragma unroll
    for (int t = 0; t < D - 2; ++t)
        if (t < nsw) issue(t);
    if (nsw >= D - 2)
        wait_vmcnt<D - 2>();   // activation and scale copies, older than the stripes
    else
        wait_vmcnt<0>();
    asm volatile("s_barrier" ::: "memory");

    const int swz = (r >> 1) & 7;
    uint32_t off[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) off[j] = r * kStripe + ((j ^ swz) << 4) + 4 * par;
    // activation dwords of chunk T hold elements 16T + 8 par + nb (and + 4)
    // in half nb & 1
    const uint32_t *my_act = (const uint32_t *)act + 4 * par + (nb >> 1);
    const uint32_t sel = (nb & 1) ? 0x03020C0Cu : 0x01000C0Cu;   // v_perm: that half -> fp32 bits
    const uint32_t shift = 4u * nb;
    const uint32_t magic = opaque_magic();

    // One or two activation rows: a stripe's activation words are read with
    // its weights, one stripe ahead; three or four: when used (the prefetched
    // words would not fit in registers).
    constexpr bool kPre = MT <= 2;
    constexpr int AB = kPre ? MT : 1;
    float acc0[MT], acc1[MT];   // chains nb and nb + 4 of the lane's half, per activation row
#pragma unroll
    for (int m = 0; m < MT; ++m) acc0[m] = acc1[m] = 0.0f;
    auto load = [&](int t, uint32_t (&x)[16], uint32_t (&av)[AB][32]) {
        const unsigned char *slot = ring + (t % D) * SLOT;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            x[2 * j] = *(const uint32_t *)(slot + off[j]);
            x[2 * j + 1] = *(const uint32_t *)(slot + off[j] + 8);
        }
        if constexpr (kPre) {
            const int st = sb + t;
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const uint32_t *ap = my_act + (size_t)m * rdw + 8 * (16 * st + u);
                    av[m][2 * u] = ap[0];
                    av[m][2 * u + 1] = ap[2];
                }
        }
    };
    auto compute = [&](int t, const uint32_t (&x)[16], const uint32_t (&av)[AB][32]) {
        const int st = sb + t;
        const int g0 = st * GPS;
#pragma unroll
        for (int gi = 0; gi < GPS; ++gi) {
#pragma unroll
            for (int u = gi * WPG; u < (gi + 1) * WPG; ++u) {
                const uint32_t v = (x[u] ^ 0x88888888u) >> shift;
                const h2 bias = {(_Float16)-1032.0f, (_Float16)-1032.0f};
                const h2 q = __builtin_bit_cast(h2, (v & 0x000F000Fu) | magic) + bias;
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    uint32_t w0, w1;
                    if constexpr (kPre) {
                        w0 = av[m][2 * u];
                        w1 = av[m][2 * u + 1];
                    } else {
                        const uint32_t *ap = my_act + (size_t)m * rdw + 8 * (16 * st + u);
                        w0 = ap[0];
                        w1 = ap[2];
                    }
                    const float a0 = __uint_as_float(__builtin_amdgcn_perm(0u, w0, sel));
                    const float a1 = __uint_as_float(__builtin_amdgcn_perm(0u, w1, sel));
                    acc0[m] = __builtin_fmaf(a0, (float)q.x, acc0[m]);
                    acc1[m] = __builtin_fmaf(a1, (float)q.y, acc1[m]);
                }
            }
            // lo + hi (lanes c < 4 read lane c + 4), then the quad sums in
            // the reference's order
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float s0 = acc0[m] + dpp_up4(acc0[m]);   // s_nb
                const float s4 = acc1[m] + dpp_up4(acc1[m]);   // s_{nb+4}
                const float h = dpp_quad_add(dpp_quad_add(s0 + s4, 0), 1);
                if (c == 0) blk[(m * 8 + r) * G + g0 + gi] = h;
                acc0[m] = 0.0f;
                acc1[m] = 0.0f;
            }
        }
    };
    uint32_t xa[16], xb[16];
    uint32_t aa[AB][32], ab[AB][32];
    if (nsw > 0) {
        if (nsw >= D - 2)
            wait_vmcnt<D - 3>();
        else
            wait_vmcnt<0>();
        load(0, xa, aa);
    }
    int t = 0;
#pragma unroll 1
    for (; t + 1 < nsw; t += 2) {
        if (t + D - 2 < nsw) issue(t + D - 2);
        if (t + D - 1 < nsw) issue(t + D - 1);
        if (t + D <= nsw)
            wait_vmcnt<D - 2>();
        else
            wait_vmcnt<0>();
        load(t + 1, xb, ab);
        compute(t, xa, aa);
        if (t + 2 < nsw) {
            if (t + D <= nsw)
                wait_vmcnt<D - 3>();
            else
                wait_vmcnt<0>();
            load(t + 2, xa, aa);
        }
        compute(t + 1, xb, ab);
    }
    if (t < nsw) compute(t, xa, aa);

    // Fold: row r's blocks in group order (kernels.c:1141-1150), by lane 8r of wave 0.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const int n = row0 + r;
    if (wave != 0 || c != 0 || n >= N) return;
    const float *sr = scl + r * G;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const float *br = blk + (m * 8 + r) * G;
        float a = 0.0f;
#pragma unroll 8
        for (int g = 0; g < G; ++g) a = __builtin_fmaf(br[g], sr[g], a);
        C[(size_t)(m0 + m) * N + n] = f32_to_bf16(a);
    }
}

template <int FMT, int MT, int D, int P>
size_t gq8_lds_bytes(int K) {
    const size_t G = (size_t)K / (FMT == F_W4G128 ? 128 : 32);
    return (size_t)P * D * 8 * kStripe + (size_t)MT * K * 2 + 8 * G * 4 + (size_t)MT * 8 * G * 4;
}

template <int FMT, int MT, int D, int P>
int launch_gq8_one(int ntiles, hipStream_t st, const uint16_t *A, const uint8_t *W, const float *S, uint16_t *C,
                   int N, int K, int m0) {
    static std::once_flag once;
    static hipError_t attr_rc = hipSuccess;
    std::call_once(once, [] {
        attr_rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_gq8_kernel<FMT, MT, D, P>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRowMaxLds);
    });
    if (attr_rc != hipSuccess) return ECPU_ERR_DEVICE;
    const size_t lds = gq8_lds_bytes<FMT, MT, D, P>(K);
    if (lds > kRowMaxLds) return ECPU_ERR_UNSUPPORTED;
    gemv_gq8_kernel<FMT, MT, D, P><<<ntiles, 64 * P, lds, st>>>(A, W, S, C, N, K, m0);
    return ECPU_OK;
}

// Eight waves with four-slot rings, or fewer waves for short rows.
template <int FMT, int MT>
int launch_gq8(int p, int ntiles, hipStream_t st, const uint16_t *A, const uint8_t *W, const float *S, uint16_t *C,
               int N, int K, int m0) {
    switch (p) {
        case 8: {
            // ring slots: five where a wave has three stripes, so all three are
            // in flight at once (2048x6144: 6.13 -> 5.90 us); four otherwise
            // (PILM_HIP_GQ8_D = 4, 5 or 8)
            const int sps = (K / 256 + 7) / 8;
            const int de = env_int("PILM_HIP_GQ8_D", sps == 3 ? 5 : 4);
            if (de == 5) return launch_gq8_one<FMT, MT, 5, 8>(ntiles, st, A, W, S, C, N, K, m0);
            if (de == 8) return launch_gq8_one<FMT, MT, 8, 8>(ntiles, st, A, W, S, C, N, K, m0);
            return launch_gq8_one<FMT, MT, 4, 8>(ntiles, st, A, W, S, C, N, K, m0);
        }
        case 4: return launch_gq8_one<FMT, MT, 8, 4>(ntiles, st, A, W, S, C, N, K, m0);
        case 2: return launch_gq8_one<FMT, MT, 8, 2>(ntiles, st, A, W, S, C, N, K, m0);
        default: return launch_gq8_one<FMT, MT, 16, 1>(ntiles, st, A, W, S, C, N, K, m0);
    }
}

template <int FMT>
int launch_gq8_mt(int mt, int p, int ntiles, hipStream_t st, const uint16_t *A, const uint8_t *W, const float *S,
                  uint16_t *C, int N, int K, int m0) {
    switch (mt) {
        case 1: return launch_gq8<FMT, 1>(p, ntiles, st, A, W, S, C, N, K, m0);
        case 2: return launch_gq8<FMT, 2>(p, ntiles, st, A, W, S, C, N, K, m0);
        case 3: return launch_gq8<FMT, 3>(p, ntiles, st, A, W, S, C, N, K, m0);
        default: return launch_gq8<FMT, 4>(p, ntiles, st, A, W, S, C, N, K, m0);
    }
}

template <int FMT>
int launch_gq_fmt(int p, int d, int mt, int ntiles, hipStream_t st, const uint16_t *A, const uint8_t *W,
                  const float *S, uint16_t *C, int N, int K, int m0) {
    switch (p) {
        case 1: return launch_gq_mt<FMT, 16, 1>(mt, ntiles, st, A, W, S, C, N, K, m0);
        case 2: return launch_gq_mt<FMT, 8, 2>(mt, ntiles, st, A, W, S, C, N, K, m0);
        case 4:
            return d == 16 ? launch_gq_mt<FMT, 16, 4>(mt, ntiles, st, A, W, S, C, N, K, m0)
                           : launch_gq_mt<FMT, 8, 4>(mt, ntiles, st, A, W, S, C, N, K, m0);
        default:   // eight waves: at most two activation rows (registers)
            if (d == 4)
                return mt == 1 ? launch_gq_one<FMT, 1, 4, 8>(ntiles, st, A, W, S, C, N, K, m0)
                               : launch_gq_one<FMT, 2, 4, 8>(ntiles, st, A, W, S, C, N, K, m0);
            return mt == 1 ? launch_gq_one<FMT, 1, 8, 8>(ntiles, st, A, W, S, C, N, K, m0)
                           : launch_gq_one<FMT, 2, 8, 8>(ntiles, st, A, W, S, C, N, K, m0);
    }
}

}  // namespace

// W8A16 GEMV of one activation row with the greedy argmax as its epilogue
// (the 64-row chain kernel at every N; 32- or 16-row tiles when there are few
// 64-row ones): no logits are written.  part holds 2 * rows_argmax_tiles(N)
// words and is 16-byte aligned, ticket must be zero.  ECPU_ERR_UNSUPPORTED (nothing launched) for K not a
// multiple of the 128-byte stripe or unaligned A / W.
int run_rows_argmax(size_t N, size_t K, const uint16_t *A, const uint8_t *W, const float *S, uint32_t *part,
                    int *ticket, uint32_t *result, size_t *out_index, float *out_value, hipStream_t st) {
    if (N == 0 || K == 0 || K % kStripe || (((uintptr_t)A | (uintptr_t)W | (uintptr_t)part) & 15) ||
        N >= ((size_t)1 << 31))
        return ECPU_ERR_UNSUPPORTED;
    RowsArgmax ao;
    ao.part = part;
    ao.ticket = ticket;
    ao.result = result;
    ao.out_index = out_index;
    ao.out_value = out_value;
    const int ntiles = (int)((N + 63) / 64);
    const int rows = ntiles >= 256 ? 64 : (ntiles >= 128 ? 32 : 16);
    const int depth = ntiles <= 256 ? 16 : (ntiles <= 512 ? 8 : 4);
    if (rows == 16) return launch_rows_argmax<16, 16>(st, A, W, S, (int)N, (int)K, ao);
    if (rows == 32) return launch_rows_argmax<16, 32>(st, A, W, S, (int)N, (int)K, ao);
    if (depth == 16) return launch_rows_argmax<16, 64>(st, A, W, S, (int)N, (int)K, ao);
    if (depth == 8) return launch_rows_argmax<8, 64>(st, A, W, S, (int)N, (int)K, ao);
    return launch_rows_argmax<4, 64>(st, A, W, S, (int)N, (int)K, ao);
}

int run_gq_norm(bool swiglu, size_t N, size_t K, const uint16_t *x, const uint16_t *res, const uint16_t *norm_w,
                uint16_t *res_out, float eps, const uint8_t *W, const float *S, uint16_t *C, hipStream_t st) {
    GqNorm na;
    na.x = x;
    na.res = res;
    na.w = norm_w;
    na.res_out = res_out;
    na.eps = eps;
    // waves per tile and ring slots (PILM_HIP_GQN_P = 2, 4 or 8, PILM_HIP_GQN_D = 3, 4 or 8); by
    // default eight waves (one stripe each at K = 2048) for the plain linear and four for
    // gate/up + SwiGLU (3 workgroups per CU instead of 2: Qwen3-1.7B decode 765 -> 794 tok/s)
    const int pe = env_int("PILM_HIP_GQN_P", swiglu ? 4 : 8);
    const int p = (pe == 2 || pe == 4) ? pe : 8;
    const int de = env_int("PILM_HIP_GQN_D", 4);
    const int d = (de == 3 || de == 8) ? de : 4;
    if (K == 0 || K % 256 || K / 8 > (size_t)kGqNormChunks * 64 * p) return ECPU_ERR_UNSUPPORTED;
    if (swiglu && N % 16) return ECPU_ERR_UNSUPPORTED;
    const int nt = swiglu ? (int)(N / 16) : (int)((N + 15) / 16);
#define PILM_GQN(SW)                                                                                         \
    (p == 2 ? (d == 8 ? launch_gq_norm<SW, 2, 8>(nt, st, W, S, C, (int)N, (int)K, na)                      \
                      : launch_gq_norm<SW, 2, 4>(nt, st, W, S, C, (int)N, (int)K, na))                     \
   : p == 4 ? (d == 3   ? launch_gq_norm<SW, 4, 3>(nt, st, W, S, C, (int)N, (int)K, na)                    \
               : d == 8 ? launch_gq_norm<SW, 4, 8>(nt, st, W, S, C, (int)N, (int)K, na)                    \
                        : launch_gq_norm<SW, 4, 4>(nt, st, W, S, C, (int)N, (int)K, na))                   \
            : (d == 3   ? launch_gq_norm<SW, 8, 3>(nt, st, W, S, C, (int)N, (int)K, na)                    \
               : d == 8 ? launch_gq_norm<SW, 8, 8>(nt, st, W, S, C, (int)N, (int)K, na)                    \
                        : launch_gq_norm<SW, 8, 4>(nt, st, W, S, C, (int)N, (int)K, na)))
    const int rc = swiglu ? PILM_GQN(true) : PILM_GQN(false);
#undef PILM_GQN
    return rc;
}

// Per-row formats on the stripe path: K a multiple of the stripe (128 int8
// or 256 int4 weights), 16-byte aligned weights and activations.
int run_rows(int fmt, size_t M, size_t N, size_t K, const void *A, const uint8_t *W, const float *S, void *C,
             hipStream_t st, const char *fn) {
    // A few activation rows: the row-broadcast kernel, every M in one launch;
    // at M = 2 only where the quad kernel would run (more than 512 16-row
    // tiles, below 65536 rows: W8A16 24576x4096 37.1 vs 52.7 us; the chain
    // kernel stays ahead below, e.g. 8192x4096 15.2 vs 19.5 us).
    const size_t qt16 = (N + 15) / 16;
    const bool rbc2 = M == 2 && qt16 > 512 && N < 65536;
    if ((M >= 3 || rbc2) && env_int("PILM_HIP_RBC", 1) != 0) return run_rbc(fmt, M, N, K, A, W, S, C, st, fn);
    // One row of W4 per-row below 4096 rows: 8-row chain tiles (measured
    // 1024x2048 4.49 -> 4.02 us, 2048x6144 8.59 -> 7.79 us; slower from 4096
    // rows on, where the 16-row tiles already cover every CU).
    if (M == 1 && fmt == F_W4ROW && env_int("PILM_HIP_W4C8", N < 4096 ? 1 : 0) != 0) {
        const int rc = launch_w4c8<16>(st, A, W, S, C, (int)N, (int)K);
        if (rc == ECPU_ERR_DEVICE) return fail(ECPU_ERR_DEVICE, "%s: raising the LDS limit of the GEMV kernel failed", fn);
        if (rc == ECPU_OK) return ECPU_OK;
    }
    // One row of a W8 format below 16384 rows: the byte-wave kernel (measured
    // W8A32 4096x4096 9.6 vs 10.4 us, 8192x4096 11.5 vs 13.5 us, 4096x12288
    // 24.1 vs 26.8 us; the quad / 64-row kernels stay ahead beyond).
    if (M == 1 && fmt != F_W4ROW && env_int("PILM_HIP_W8B", N < 16384 ? 1 : 0) != 0) {
        const int rc = fmt == F_W8A32 ? launch_w8b<F_W8A32>(st, A, W, S, C, (int)N, (int)K)
                                      : launch_w8b<F_W8A16>(st, A, W, S, C, (int)N, (int)K);
        if (rc != ECPU_OK) return fail(ECPU_ERR_DEVICE, "%s: raising the LDS limit of the GEMV kernel failed", fn);
        return ECPU_OK;
    }
    // Few 16-row tiles: the chain kernel (several SIMDs per tile).
    const int qt_all = (int)((N + 15) / 16);
    int cs = env_int("PILM_HIP_CS", -1);
    if (cs < 0) cs = qt_all <= 512 ? (fmt == F_W4ROW ? (qt_all <= 256 ? 4 : 2) : 2) : 0;
    if (fmt != F_W4ROW && cs == 4) cs = 2;
    if (cs == 2 || cs == 4) {
        int per = 0;
        switch (fmt) {
            case F_W8A32: per = chain_rows_per_launch<F_W8A32, 2>((int)K); break;
            case F_W8A16: per = chain_rows_per_launch<F_W8A16, 2>((int)K); break;
            default: per = cs == 4 ? chain_rows_per_launch<F_W4ROW, 4>((int)K) : chain_rows_per_launch<F_W4ROW, 2>((int)K);
        }
        if (per > 0) {
            for (size_t m0 = 0; m0 < M; m0 += per) {
                const int mt = (int)std::min<size_t>(per, M - m0);
                int rc;
                switch (fmt) {
                    case F_W8A32: rc = launch_chain_mt<F_W8A32, 2>(mt, qt_all, st, A, W, S, C, (int)N, (int)K, (int)m0); break;
                    case F_W8A16: rc = launch_chain_mt<F_W8A16, 2>(mt, qt_all, st, A, W, S, C, (int)N, (int)K, (int)m0); break;
                    default:
                        rc = cs == 4 ? launch_chain_mt<F_W4ROW, 4>(mt, qt_all, st, A, W, S, C, (int)N, (int)K, (int)m0)
                                     : launch_chain_mt<F_W4ROW, 2>(mt, qt_all, st, A, W, S, C, (int)N, (int)K, (int)m0);
                }
                if (rc == ECPU_ERR_DEVICE)
                    return fail(ECPU_ERR_DEVICE, "%s: raising the LDS limit of the GEMV kernel failed", fn);
                if (rc != ECPU_OK) return fail(ECPU_ERR_DEVICE, "%s: chain kernel launch does not fit in LDS", fn);
            }
            return ECPU_OK;
        }
    }
    // Below 65536 rows (16384 for fp32 activations) the 16-row quad kernel
    // (measured faster there); above, the 64-row chain-split kernel, whose
    // scalar activations cost less VALU (W8A32 24576x4096: 27.0 vs 40.9 us).
    if (env_int("PILM_HIP_QUAD", N < (fmt == F_W8A32 ? 16384u : 65536u) ? 1 : 0) != 0) {
        // 16-row tiles; one wave per workgroup while there are few tiles (more
        // CUs), four beyond (fewer copies of the activations).
        const int qt = (int)((N + 15) / 16);
        const int wpb = qt >= 2048 ? 4 : 1;
        int depth = (qt <= 512) ? 16 : 8;
        const int env_depth = env_int("PILM_HIP_RING", 0);
        if (env_depth == 4 || env_depth == 8 || env_depth == 16) depth = env_depth;
        bool ok = true;
        for (size_t m0 = 0; m0 < M && ok; m0 += 4) {
            const int mt = (int)std::min<size_t>(4, M - m0);
            int rc;
            switch (fmt) {
                case F_W8A32: rc = launch_quad_fmt<F_W8A32>(depth, mt, wpb, qt, st, A, W, S, C, (int)M, (int)N, (int)K, (int)m0); break;
                case F_W8A16: rc = launch_quad_fmt<F_W8A16>(depth, mt, wpb, qt, st, A, W, S, C, (int)M, (int)N, (int)K, (int)m0); break;
                default: rc = launch_quad_fmt<F_W4ROW>(depth, mt, wpb, qt, st, A, W, S, C, (int)M, (int)N, (int)K, (int)m0); break;
            }
            if (rc == ECPU_ERR_DEVICE) return fail(ECPU_ERR_DEVICE, "%s: raising the LDS limit of the GEMV kernel failed", fn);
            if (rc != ECPU_OK) {
                if (m0 != 0) return fail(ECPU_ERR_DEVICE, "%s: activation staging does not fit in LDS", fn);
                ok = false;   // activations too long for LDS: chain-split kernel below
            }
        }
        if (ok) return ECPU_OK;
    }
    const int ntiles = (int)((N + 63) / 64);
    // Tile height: a CU streams only ~25-30 GB/s, so fewer than 256 tiles of
    // 64 rows would leave CUs idle; 16- or 32-row tiles (the other lanes idle)
    // spread the rows over more CUs.  Ring depth: the slots of all resident
    // tiles share the 160 KB of LDS: 16 while the tiles fit on the CUs at once,
    // 8 up to two tiles per CU, 4 beyond.
    int rows = ntiles >= 256 ? 64 : (ntiles >= 128 ? 32 : 16);
    const int env_rows = env_int("PILM_HIP_ROWTILE", 0);
    if (env_rows == 16 || env_rows == 32 || env_rows == 64) rows = env_rows;
    int depth = ntiles <= 256 ? 16 : (ntiles <= 512 ? 8 : 4);
    const int env_depth = env_int("PILM_HIP_RING", 0);
    if (env_depth == 4 || env_depth == 8 || env_depth == 16) depth = env_depth;
    for (size_t m0 = 0; m0 < M; m0 += 4) {
        const int mt = (int)std::min<size_t>(4, M - m0);
        int rc;
        switch (fmt) {
            case F_W8A32: rc = launch_rows_fmt<F_W8A32>(rows, depth, mt, st, A, W, S, C, (int)M, (int)N, (int)K, (int)m0); break;
            case F_W8A16: rc = launch_rows_fmt<F_W8A16>(rows, depth, mt, st, A, W, S, C, (int)M, (int)N, (int)K, (int)m0); break;
            default: rc = launch_rows_fmt<F_W4ROW>(rows, depth, mt, st, A, W, S, C, (int)M, (int)N, (int)K, (int)m0); break;
        }
        if (rc != ECPU_OK) return fail(ECPU_ERR_DEVICE, "%s: raising the LDS limit of the GEMV kernel failed", fn);
    }
    return ECPU_OK;
}

// Gate/up half of the fused W4 SwiGLU (kernels.c:1623-1659) for M = 1:
// hidden[i] = bf16(silu(g_i) * u_i) from one pass over the 2I gate/up rows.
// ECPU_ERR_UNSUPPORTED (nothing launched) when the stripe kernel cannot take
// the shape: K not a multiple of 256, unaligned A or W, or activations too
// long for LDS.
int run_swiglu_gate_up(size_t I, size_t K, const uint16_t *A, const uint8_t *W, const float *S, uint16_t *hidden,
                       hipStream_t st) {
    if (I == 0) return ECPU_OK;
    if (K == 0 || K % 256 != 0 || (((uintptr_t)A | (uintptr_t)W) & 15) != 0 || I >= ((size_t)1 << 30))
        return ECPU_ERR_UNSUPPORTED;
    const int nt = (int)((I + 7) / 8);
    const int wpb = nt >= 2048 ? 4 : 1;
    int depth = nt <= 512 ? 16 : 8;
    const int env_depth = env_int("PILM_HIP_RING", 0);
    if (env_depth == 8 || env_depth == 16) depth = env_depth;
    if (depth == 16)
        return launch_quad_one<F_W4ROW, 1, 16, true>(wpb, nt, st, A, W, S, hidden, 1, (int)I, (int)K, 0);
    return launch_quad_one<F_W4ROW, 1, 8, true>(wpb, nt, st, A, W, S, hidden, 1, (int)I, (int)K, 0);
}

// Group formats (fmt 3 W4A16 g128, 4 g32) on the group-quad kernel: K a
// multiple of 256, 16-byte aligned A and W.  P waves per 16-row tile divide
// its stripes: enough to give ~256 waves when the tiles are few.
// ECPU_ERR_UNSUPPORTED (nothing launched) when LDS cannot hold one row.
int run_group_quad(int fmt, size_t M, size_t N, size_t K, const void *A, const uint8_t *W, const float *S, void *C,
                   hipStream_t st, const char *fn) {
    const int ntiles = (int)((N + 15) / 16);
    const int ns = (int)(K / 256);
    // 8-row tiles: one or two activation rows with fewer 16-row tiles than
    // CUs, more rows up to 6144 output rows (g128 4096x2048 M=4 7.8 vs 8.9
    // us; M=2 7.8 vs 5.8, so not there), in launches of up to four rows
    // (as many as LDS holds).
    if (env_int("PILM_HIP_GQ8", (M <= 2 ? ntiles < 256 : ntiles <= 384) ? 1 : 0) != 0) {
        int p = 8;
        while (p > 1 && ns < p) p /= 2;
        const size_t G = K / (fmt == F_W4G128 ? 128 : 32);
        const int d = p == 8 ? 4 : (p == 1 ? 16 : 8);
        int per = 4;
        while (per > 0 && (size_t)p * d * 8 * kStripe + (size_t)per * K * 2 + 8 * G * 4 + (size_t)per * 8 * G * 4 > kRowMaxLds)
            --per;
        const int nt8 = (int)((N + 7) / 8);
        for (size_t m0 = 0; per > 0 && m0 < M; m0 += per) {
            const int mt = (int)std::min<size_t>(per, M - m0);
            const int rc = fmt == F_W4G128
                               ? launch_gq8_mt<F_W4G128>(mt, p, nt8, st, (const uint16_t *)A, W, S, (uint16_t *)C,
                                                         (int)N, (int)K, (int)m0)
                               : launch_gq8_mt<F_W4G32>(mt, p, nt8, st, (const uint16_t *)A, W, S, (uint16_t *)C,
                                                        (int)N, (int)K, (int)m0);
            if (rc == ECPU_ERR_DEVICE) return fail(ECPU_ERR_DEVICE, "%s: raising the LDS limit of the GEMV kernel failed", fn);
            if (rc != ECPU_OK) return fail(ECPU_ERR_DEVICE, "%s: 8-row group-quad launch does not fit in LDS", fn);
        }
        if (per > 0) return ECPU_OK;
        // (rows too long for LDS: the 16-row kernel below)
    }
    // Eight waves per tile for one or two activation rows (the eight-wave
    // kernels hold two in registers; measured faster than four at every
    // Qwen3 shape, e.g. 6144x2048 5.5 vs 6.1 us, 8192x4096 8.9 vs 11.0 us),
    // four beyond.  Every wave gets a stripe.
    int p = M <= 2 ? 8 : 4, d = 8;
    const int env_p = env_int("PILM_HIP_GQ_P", 0), env_d = env_int("PILM_HIP_GQ_D", 0);
    if (env_p == 1 || env_p == 2 || env_p == 4 || env_p == 8) p = env_p;
    while (p > 1 && ns < p) p /= 2;
    // Ring depth: 16 slots for one wave, 8 for four (16 on request), 4 for
    // eight (the same bytes in flight per CU as four waves of 8, half the LDS,
    // measured faster: 1.7B decode step 1.070 -> 1.058 ms; 8 on request).
    d = p == 1 ? 16 : (p == 4 ? (env_d == 16 ? 16 : 8) : (p == 8 ? (env_d == 8 ? 8 : 4) : 8));
    // activation rows per launch: the largest of 4, 2, 1 that fits LDS
    auto fits = [&](int mt) {
        const size_t G = K / (fmt == F_W4G128 ? 128 : 32);
        return (size_t)p * d * 2048 + (size_t)mt * K * 2 + 16 * G * 4 + (size_t)mt * 16 * G * 4 <= kRowMaxLds;
    };
    // Long rows (K = 12288 with group 32) may leave no room for the rings:
    // fewer waves rather than the exact kernel.
    if (p == 8 && !fits(1)) d = 4;
    while (p > 1 && !fits(1)) {
        p /= 2;
        d = p == 1 ? 16 : 8;
    }
    const int per = (p < 8 && fits(4)) ? 4 : (fits(2) ? 2 : (fits(1) ? 1 : 0));
    if (per == 0) return ECPU_ERR_UNSUPPORTED;
    for (size_t m0 = 0; m0 < M; m0 += per) {
        const int mt = (int)std::min<size_t>(per, M - m0);
        const int rc = fmt == F_W4G128
                           ? launch_gq_fmt<F_W4G128>(p, d, mt, ntiles, st, (const uint16_t *)A, W, S,
                                                     (uint16_t *)C, (int)N, (int)K, (int)m0)
                           : launch_gq_fmt<F_W4G32>(p, d, mt, ntiles, st, (const uint16_t *)A, W, S,
                                                    (uint16_t *)C, (int)N, (int)K, (int)m0);
        if (rc == ECPU_ERR_DEVICE) return fail(ECPU_ERR_DEVICE, "%s: raising the LDS limit of the GEMV kernel failed", fn);
        if (rc != ECPU_OK) return fail(ECPU_ERR_DEVICE, "%s: group-quad launch does not fit in LDS", fn);
    }
    return ECPU_OK;
}

}  // namespace pilm
