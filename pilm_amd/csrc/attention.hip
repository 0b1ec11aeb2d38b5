// Paged attention of one sequence on the GPU: the step FullAttention.forward
// takes after q_norm / k_norm / rope (src/models/qwen3/attention.py:95-139)
// over the block-paged cache of src/runtime/kvcache/physical_kv.py:11-81,
// with the reference's roundings: bf16 scores of an fp32 dot product, a bf16
// product with 1/sqrt(D), softmax in fp32, weights rounded to bf16, a bf16
// P.V of fp32 sums, and the bf16 sigmoid gate.
//
// Two launches per group of query rows:
//   attn_scores_kernel  grid (chunks of 256 positions, kv heads): lane =
//       position; the position's key row (from the cache through the block
//       table, or the step's own new rows, which it also writes into the
//       cache) is dotted with every query row that reads this kv head (the
//       heads of the GQA group x the step's tokens, held in LDS and read as
//       broadcasts).  Scores go to scratch as bf16; each chunk also leaves
//       its (max, sum of exp(score - max)) per row.
//   attn_pv_kernel      same grid: every workgroup folds the chunk
//       statistics into the row's max and sum (the same order in each, so
//       the same values), forms the bf16 weights of its chunk, and
//       accumulates P.V with lane = head-dim column (a wave reads one value
//       row per instruction); waves meet in LDS in wave order, chunks in a
//       global fold in chunk order by the last workgroup of the kv head (a
//       ticket), which rounds, applies the gate and stores.
// K and V are read once from HBM per kv head; that is the kernel's roofline.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdint>
#include <mutex>
#include <type_traits>

#include "gemv_device.h"
#include "internal.h"

namespace pilm {
namespace {

constexpr int kChunk = 256;    // positions per workgroup (one per thread of the score pass)
constexpr int kMaxRows = 32;   // query rows per kv head and launch (heads of the group x tokens)

struct AttnArgs {
    const uint16_t *q;       // [S_total, H, D]
    const uint16_t *k_new;   // [S_total, Hkv, D]
    const uint16_t *v_new;
    uint16_t *k_cache;       // [NB, BS, Hkv, D] or null
    uint16_t *v_cache;
    const int32_t *block_ids;
    const uint16_t *gate;    // (s, h, d) at gate[(s * H + h) * gate_stride + d], or null
    uint16_t *out;           // [S_total, H * D]
    uint16_t *scores;        // [Hkv][RB][Lp] bf16
    float *stats;            // [nchunk][Hkv][RB][2]: chunk max, chunk sum
    float *gstat;            // [Hkv][RB][2]: row max, 1 / row sum
    float *part;             // [ngroups][Hkv][RB][D]: P.V sums of each group of chunks
    int *tickets;            // [2 * Hkv], zero between launches (P.V fold, statistics fold)
    int S;                   // query rows of this launch (R = S * rep)
    int s0;                  // first of them within the step
    int H, Hkv, rep;
    int new0;                // position of the step's first new row: cache_len - S_total
    int L;                   // positions this launch reads: new0 + s0 + S
    int Lp;                  // L rounded up to whole chunks
    int nchunk;
    int fold_in_pv;          // few chunks: every P.V wave folds the chunk statistics itself
    int cpw;                 // chunks per P.V workgroup
    int ngroups;             // P.V workgroups per kv head: ceil(nchunk / cpw)
    int BS, NB;
    int write_cache;         // store this launch's rows (positions new0 + s0 ..) into the caches
    int gate_stride;
    float scale;             // (float)(1 / sqrt(D)), as the reference's Python float meets bf16
};

// Global-memory views of the row pointers: loads through them are global_load
// (vector memory counter only), not flat loads, which would also hold up
// every LDS wait behind them.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T *gbl(const T *p) {
    return (const __attribute__((address_space(1))) T *)p;
}
template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T *gbl_w(T *p) {
    return (__attribute__((address_space(1))) T *)p;
}

__device__ __forceinline__ float bf16_round(float x) { return __uint_as_float((uint32_t)f32_to_bf16(x) << 16); }
__device__ __forceinline__ float bf16_bits(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }

// Row of position j of kv head kvh: the step's new rows come from its own K / V.
template <int D>
__device__ __forceinline__ const uint16_t *kv_row(const AttnArgs &a, const uint16_t *cache, const uint16_t *fresh,
                                                  int j, int kvh) {
    if (j >= a.new0) return fresh + ((size_t)(j - a.new0) * a.Hkv + kvh) * D;
    const int b = min(max(a.block_ids[j / a.BS], 0), a.NB - 1);
    return cache + (((size_t)b * a.BS + j % a.BS) * a.Hkv + kvh) * D;
}

template <int D>
__device__ __forceinline__ uint16_t *cache_row(const AttnArgs &a, uint16_t *cache, int j, int kvh) {
    const int b = min(max(a.block_ids[j / a.BS], 0), a.NB - 1);
    return cache + (((size_t)b * a.BS + j % a.BS) * a.Hkv + kvh) * D;
}

// exp for the softmax and the gate: the device library's single-precision
// exp (ALU only, within 1 ulp).  The reference's is torch's vectorized CPU
// exp, not a correctly rounded one either; either way the weights are then
// rounded to bf16.
__device__ __forceinline__ float att_exp(float x) { return expf(x); }

// Wave reductions in a fixed order with DPP inside each 16-lane row (quad
// swaps, then rotations by 4 and 8) and the four row results by v_readlane:
// ALU operations only, no LDS round trip.  The result is wave-uniform.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f(float x, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}

__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp_f<0xB1>(x));    // quad_perm [1,0,3,2]
    x = fmaxf(x, dpp_f<0x4E>(x));    // quad_perm [2,3,0,1]
    x = fmaxf(x, dpp_f<0x124>(x));   // row_ror:4
    x = fmaxf(x, dpp_f<0x128>(x));   // row_ror:8
    return fmaxf(fmaxf(lane_f(x, 0), lane_f(x, 16)), fmaxf(lane_f(x, 32), lane_f(x, 48)));
}

__device__ __forceinline__ float wave_sum(float x) {
    x = x + dpp_f<0xB1>(x);
    x = x + dpp_f<0x4E>(x);
    x = x + dpp_f<0x124>(x);
    x = x + dpp_f<0x128>(x);
    return (lane_f(x, 0) + lane_f(x, 16)) + (lane_f(x, 32) + lane_f(x, 48));
}

template <int D, int RB>
__global__ __launch_bounds__(256) void attn_scores_kernel(AttnArgs a) {
    __shared__ float qs[RB * D];
    __shared__ float wmax[4][RB], wsum[4][RB], cmax[RB];
    __shared__ int last;
    const int chunk = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    // row group z of the kv head: rows rz0 .. rz0 + RB - 1 of the launch's
    // S * rep; scratch is indexed by kz (kv head and row group) over HZ
    const int rz0 = blockIdx.z * RB, kz = kvh * gridDim.z + blockIdx.z, HZ = a.Hkv * gridDim.z;
    const int R = min(RB, a.S * a.rep - rz0);
    // query rows r = s * rep + i (head kvh * rep + i, token s0 + s) as fp32
    for (int e = tid; e < RB * D; e += 256) {
        const int r = e / D, d = e - r * D;
        float v = 0.0f;
        if (r < R) {
            const int s = (rz0 + r) / a.rep, h = kvh * a.rep + (rz0 + r - s * a.rep);
            v = bf16_bits(a.q[((size_t)(a.s0 + s) * a.H + h) * D + d]);
        }
        qs[e] = v;
    }
    __syncthreads();

    const int j = chunk * kChunk + tid;
    const bool valid = j < a.L;
    float acc[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) acc[r] = 0.0f;
    if (valid) {
        const auto *kp = gbl((const u32x4 *)kv_row<D>(a, a.k_cache, a.k_new, j, kvh));
        auto *dst = (a.write_cache && blockIdx.z == 0 && j >= a.new0 + a.s0) ? gbl_w((u32x4 *)cache_row<D>(a, a.k_cache, j, kvh)) : nullptr;
        // The loads of a row go out a whole 128-byte line at a time: issued
        // two by two with the dot in between, a line's later 16-byte pieces
        // were asked for after other waves' traffic had evicted it from L2,
        // and K came from HBM 1.9 times (8B decode, 32768 positions).  The
        // cache store sits outside the dot: inside it, its branch split the
        // line into blocks and the compiler hoisted every LDS read of q
        // ahead of the FMAs (272 VGPRs at 4 rows, 76 now).
        constexpr int kLine = 8;
#pragma unroll 1
        for (int c0 = 0; c0 < D / 8; c0 += kLine) {
            u32x4 kv[kLine];
#pragma unroll
            for (int i = 0; i < kLine; ++i) kv[i] = kp[c0 + i];
            if (dst) {
#pragma unroll
                for (int i = 0; i < kLine; ++i) dst[c0 + i] = kv[i];
            }
#pragma unroll
            for (int i = 0; i < kLine; ++i) {
                const int c = c0 + i;
                const uint32_t w[4] = {kv[i].x, kv[i].y, kv[i].z, kv[i].w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const float k0 = bf16_lo(w[t]), k1 = bf16_hi(w[t]);
#pragma unroll
                    for (int r = 0; r < RB; ++r) {
                        acc[r] = __builtin_fmaf(qs[r * D + 8 * c + 2 * t], k0, acc[r]);
                        acc[r] = __builtin_fmaf(qs[r * D + 8 * c + 2 * t + 1], k1, acc[r]);
                    }
                }
                // (keeps the LDS reads of q beside their FMAs, not all
                // hoisted ahead of the line)
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    // attention.py:128-134: bf16 bmm output, times the scale in bf16, causal mask
    float sc[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const bool seen = valid && r < R && j <= a.new0 + a.s0 + (rz0 + r) / a.rep;
        sc[r] = seen ? bf16_round(bf16_round(acc[r]) * a.scale) : -__builtin_inff();
        if (r < R) a.scores[((size_t)kz * RB + r) * a.Lp + j] = f32_to_bf16(sc[r]);
    }
    // chunk statistics: max, then sum of exp(score - max)
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const float m = wave_max(sc[r]);
        if (lane == 0) wmax[wave][r] = m;
    }
    __syncthreads();
    if (tid < RB) cmax[tid] = fmaxf(fmaxf(wmax[0][tid], wmax[1][tid]), fmaxf(wmax[2][tid], wmax[3][tid]));
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const float m = cmax[r];
        const float e = sc[r] == -__builtin_inff() ? 0.0f : att_exp(sc[r] - m);
        const float l = wave_sum(e);
        if (lane == 0) wsum[wave][r] = l;
    }
    __syncthreads();
    if (a.fold_in_pv) {
        if (tid < R) {
            float *st = a.stats + (((size_t)chunk * HZ + kz) * RB + tid) * 2;
            st[0] = cmax[tid];
            st[1] = ((wsum[0][tid] + wsum[1][tid]) + wsum[2][tid]) + wsum[3][tid];
        }
        return;
    }
    // The chunk statistics leave as agent-scope stores; the last chunk of
    // the kv head (ticket) folds them into the row's max and 1 / sum: wave w
    // takes rows w, w + 4, ..; lane c chunks c, c + 64, .. in order, then the
    // lanes meet in a fixed butterfly.
    if (tid < R) {
        float *st = a.stats + (((size_t)chunk * HZ + kz) * RB + tid) * 2;
        __hip_atomic_store(st, cmax[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(st + 1, ((wsum[0][tid] + wsum[1][tid]) + wsum[2][tid]) + wsum[3][tid], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    wait_vmcnt<0>();
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(a.tickets + HZ + kz, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               a.nchunk - 1;
    __syncthreads();
    if (!last) return;
    const size_t cstride = (size_t)HZ * RB * 2;
    for (int r = wave; r < R; r += 4) {
        const float *st = a.stats + ((size_t)kz * RB + r) * 2;
        float m = -__builtin_inff();
        for (int c = lane; c < a.nchunk; c += 64)
            m = fmaxf(m, __hip_atomic_load(st + c * cstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        m = wave_max(m);
        float l = 0.0f;
        for (int c = lane; c < a.nchunk; c += 64) {
            const float mc = __hip_atomic_load(st + c * cstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float lc = __hip_atomic_load(st + c * cstride + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (mc != -__builtin_inff()) l = l + lc * att_exp(mc - m);
        }
        l = wave_sum(l);
        if (lane == 0) {
            float *gs = a.gstat + ((size_t)kz * RB + r) * 2;
            gs[0] = m;
            gs[1] = 1.0f / l;
        }
    }
    if (tid == 0) __hip_atomic_store(a.tickets + HZ + kz, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int D, int RB>
constexpr size_t pv_lds_bytes() {
    return ((size_t)RB * kChunk + 3 * (size_t)RB * D + 4 * 2 * RB) * sizeof(float);
}

template <int D, int RB>
__global__ __launch_bounds__(256) void attn_pv_kernel(AttnArgs a) {
    constexpr int E = D / 64;                 // head-dim columns per lane
    constexpr int kBatch = E == 4 ? 32 : 64;  // value rows in flight per wave
    extern __shared__ float lds[];
    float *p = lds;                           // [RB][kChunk] bf16 weights as fp32 (wave w: columns 64w..)
    float *red = p + RB * kChunk;             // [3][RB][D] sums of waves 1..3
    const int grp = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    float *gm = red + 3 * RB * D + wave * 2 * RB;   // [RB] row max, then [RB] 1 / row sum (per wave)
    float *ginv = gm + RB;
    const int rz0 = blockIdx.z * RB, kz = kvh * gridDim.z + blockIdx.z, HZ = a.Hkv * gridDim.z;   // (row group)
    const int R = min(RB, a.S * a.rep - rz0);
    const float ninf = -__builtin_inff();
    const int t0 = wave * 64;
    if (lane < R) {
        if (a.fold_in_pv) {
            // (up to 8 chunks: the row's max and sum folded here, in chunk order)
            const float *st = a.stats + ((size_t)kz * RB + lane) * 2;
            const size_t cstride = (size_t)HZ * RB * 2;
            float mc[8], lc[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                mc[c] = c < a.nchunk ? st[c * cstride] : ninf;
                lc[c] = c < a.nchunk ? st[c * cstride + 1] : 0.0f;
            }
            float m = ninf;
#pragma unroll
            for (int c = 0; c < 8; ++c) m = fmaxf(m, mc[c]);
            float l = 0.0f;
#pragma unroll
            for (int c = 0; c < 8; ++c)
                if (mc[c] != ninf) l = l + lc[c] * att_exp(mc[c] - m);
            gm[lane] = m;
            ginv[lane] = 1.0f / l;
        } else {
            const float *gs = a.gstat + ((size_t)kz * RB + lane) * 2;
            gm[lane] = gs[0];
            ginv[lane] = gs[1];
        }
    }
    __builtin_amdgcn_wave_barrier();   // (LDS is in order within the wave; keep the compiler from reordering)

    // Each wave works alone until the waves' sums meet.  Per chunk of the
    // group: lane l looks up the value row of position t0 + l (storing this
    // launch's new rows into the cache), the wave's value loads go out, lane
    // l forms that position's weights, then the FMAs run in position order.
    float acc[RB][E];
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int e = 0; e < E; ++e) acc[r][e] = 0.0f;
    uint64_t myrow_bits = 0;
    int jn = 0;
    // lane t's row pointer as a wave-uniform value (v_readlane: no LDS trip)
    auto row_of = [&](int t) -> const uint16_t * {
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)myrow_bits, t);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(myrow_bits >> 32), t);
        return (const uint16_t *)(uintptr_t)(((uint64_t)hi << 32) | lo);
    };
    // raw value words, unpacked at their FMAs (unpacking at the load would
    // make the compiler wait for each load in turn)
    typedef std::conditional_t<E == 1, uint16_t, std::conditional_t<E == 2, uint32_t, u32x2>> Raw;
    Raw raw[kBatch];
    auto load_batch = [&](int tb) {
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            // every lane's row is a valid one (positions past the end read
            // the last position's); their weights are zero and their values dropped
            raw[u] = *gbl((const Raw *)(row_of(tb + u) + E * lane));
        }
    };
    auto value = [&](int tb, int u, float (&v)[E]) {
        const bool in = tb + u < jn;
        if constexpr (E == 1) {
            v[0] = in ? bf16_bits(raw[u]) : 0.0f;
        } else if constexpr (E == 2) {
            v[0] = in ? bf16_lo(raw[u]) : 0.0f;
            v[1] = in ? bf16_hi(raw[u]) : 0.0f;
        } else {
            v[0] = in ? bf16_lo(raw[u].x) : 0.0f;
            v[1] = in ? bf16_hi(raw[u].x) : 0.0f;
            v[2] = in ? bf16_lo(raw[u].y) : 0.0f;
            v[3] = in ? bf16_hi(raw[u].y) : 0.0f;
        }
    };
    const int c_end = min(a.nchunk, (grp + 1) * a.cpw);
    for (int chunk = grp * a.cpw; chunk < c_end; ++chunk) {
        jn = min(64, a.L - (chunk * kChunk + t0));   // this wave's positions (may be <= 0)
        const int jl = chunk * kChunk + t0 + lane;
        const uint16_t *myrow = kv_row<D>(a, a.v_cache, a.v_new, min(jl, a.L - 1), kvh);
        if (jl < a.L && a.write_cache && blockIdx.z == 0 && jl >= a.new0 + a.s0) {
            auto *dst = gbl_w((u32x4 *)cache_row<D>(a, a.v_cache, jl, kvh));
#pragma unroll 4
            for (int c = 0; c < D / 8; ++c) dst[c] = gbl((const u32x4 *)myrow)[c];
        }
        myrow_bits = (uint64_t)(uintptr_t)myrow;
        if (jn > 0) load_batch(0);
        // attention.py:136: softmax in fp32 (exp(x - max) * (1 / sum)), weights to bf16
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            float w = 0.0f;
            if (r < R) {
                const float sc = bf16_bits(a.scores[((size_t)kz * RB + r) * a.Lp + chunk * kChunk + t0 + lane]);
                if (sc != ninf) w = bf16_round(att_exp(sc - gm[r]) * ginv[r]);
            }
            p[r * kChunk + t0 + lane] = w;
        }
        __builtin_amdgcn_wave_barrier();
        // attention.py:137: P.V over the wave's positions in order
        for (int tb = 0; tb < jn; tb += kBatch) {
            if (tb > 0) load_batch(tb);
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                float v[E];
                value(tb, u, v);
#pragma unroll
                for (int r = 0; r < RB; ++r) {
                    const float w = p[r * kChunk + t0 + tb + u];
#pragma unroll
                    for (int e = 0; e < E; ++e) acc[r][e] = __builtin_fmaf(w, v[e], acc[r][e]);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();   // (the next chunk's weights reuse the wave's columns)
    }
    if (wave != 0) {
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int e = 0; e < E; ++e) red[((wave - 1) * RB + r) * D + E * lane + e] = acc[r][e];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int d = E * lane + e;
            acc[r][e] = ((acc[r][e] + red[r * D + d]) + red[(RB + r) * D + d]) + red[(2 * RB + r) * D + d];
        }

    auto store = [&](int r, int d, float x) {
        // attention.py:137-139: bf16 P.V, rows (s, h), bf16(out * bf16(sigmoid(gate)))
        const int s = (rz0 + r) / a.rep, h = kvh * a.rep + (rz0 + r - s * a.rep);
        const size_t row = (size_t)(a.s0 + s) * a.H + h;
        uint16_t o = f32_to_bf16(x);
        if (a.gate) {
            const float g = bf16_bits(a.gate[row * a.gate_stride + d]);
            const float sig = bf16_round(1.0f / (1.0f + att_exp(-g)));
            o = f32_to_bf16(bf16_bits(o) * sig);
        }
        a.out[row * D + d] = o;
    };
    if (a.ngroups == 1) {
#pragma unroll
        for (int r = 0; r < RB; ++r)
            if (r < R)
#pragma unroll
                for (int e = 0; e < E; ++e) store(r, E * lane + e, acc[r][e]);
        return;
    }
    // Group sums leave as agent-scope stores; once they have completed the
    // wave takes the kv head's ticket, and the last group folds them all in
    // group order with agent-scope loads.
    float *mine = a.part + ((size_t)grp * HZ + kz) * RB * D;
#pragma unroll
    for (int r = 0; r < RB; ++r)
        if (r < R)
#pragma unroll
            for (int e = 0; e < E; ++e)
                __hip_atomic_store(mine + r * D + E * lane + e, acc[r][e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    wait_vmcnt<0>();
    int ticket = 0;
    if (lane == 0) ticket = __hip_atomic_fetch_add(a.tickets + kz, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ticket = __builtin_amdgcn_readfirstlane(ticket);
    if (ticket != a.ngroups - 1) return;
    const size_t gstride = (size_t)HZ * RB * D;
    const float *base = a.part + (size_t)kz * RB * D;
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int d = E * lane + e;
            // group sums in group order, loaded 16 at a time
            float x = 0.0f;
            for (int g0 = 0; g0 < a.ngroups; g0 += 16) {
                float y[16];
#pragma unroll
                for (int u = 0; u < 16; ++u)
                    y[u] = g0 + u < a.ngroups ? __hip_atomic_load(base + (g0 + u) * gstride + r * D + d,
                                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                              : 0.0f;
#pragma unroll
                for (int u = 0; u < 16; ++u)
                    if (g0 + u < a.ngroups) x += y[u];
            }
            store(r, d, x);
        }
    if (lane == 0) __hip_atomic_store(a.tickets + kz, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Short contexts (L <= 512 positions, RB x D <= 1024): the whole step in
// one workgroup of eight waves per kv head and one launch.  Thread t owns
// position t: it forms its scores (as the score pass) and keeps its softmax
// weights and value-row pointer in registers; wave w then runs P.V over
// exactly the 64 positions its lanes own (weights and row pointers by
// v_readlane), so no scratch, ticket or second launch is needed.  Row max and
// sum meet through LDS in a fixed order.
constexpr int kSmallL = 512;
constexpr int kSmallWaves = kSmallL / 64;

template <int D, int RB>
__global__ __launch_bounds__(kSmallL) void attn_small_kernel(AttnArgs a) {
    constexpr int E = D / 64;
    constexpr int W = kSmallWaves;
    typedef std::conditional_t<E == 1, uint16_t, std::conditional_t<E == 2, uint32_t, u32x2>> Raw;
    __shared__ float qs[RB * D];
    __shared__ float wred[W][RB], rmax[RB], rinv[RB];
    __shared__ float red[(W - 1) * RB * D];
    const int kvh = blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int rz0 = blockIdx.y * RB;   // row group
    const int R = min(RB, a.S * a.rep - rz0);
    const float ninf = -__builtin_inff();
    for (int e = tid; e < RB * D; e += kSmallL) {
        const int r = e / D, d = e - r * D;
        float v = 0.0f;
        if (r < R) {
            const int s = (rz0 + r) / a.rep, h = kvh * a.rep + (rz0 + r - s * a.rep);
            v = bf16_bits(a.q[((size_t)(a.s0 + s) * a.H + h) * D + d]);
        }
        qs[e] = v;
    }
    __syncthreads();

    // scores of position tid (attention.py:128-134)
    const int j = tid;
    const bool valid = j < a.L;
    const uint64_t vrow = (uint64_t)(uintptr_t)kv_row<D>(a, a.v_cache, a.v_new, min(j, a.L - 1), kvh);
    float sc[RB];
    {
        float acc[RB];
#pragma unroll
        for (int r = 0; r < RB; ++r) acc[r] = 0.0f;
        if (valid) {
            const auto *kp = gbl((const u32x4 *)kv_row<D>(a, a.k_cache, a.k_new, j, kvh));
            const bool fresh = a.write_cache && blockIdx.y == 0 && j >= a.new0 + a.s0;
            auto *kdst = fresh ? gbl_w((u32x4 *)cache_row<D>(a, a.k_cache, j, kvh)) : nullptr;
            if (fresh) {
                auto *vdst = gbl_w((u32x4 *)cache_row<D>(a, a.v_cache, j, kvh));
                const auto *vsrc = gbl((const u32x4 *)(uintptr_t)vrow);
#pragma unroll 4
                for (int c = 0; c < D / 8; ++c) vdst[c] = vsrc[c];
            }
            // a whole 128-byte line of the key row per batch of loads, the
            // cache store outside the dot (as in the score pass)
            constexpr int kLine = 8;
#pragma unroll 1
            for (int c0 = 0; c0 < D / 8; c0 += kLine) {
                u32x4 kv[kLine];
#pragma unroll
                for (int i = 0; i < kLine; ++i) kv[i] = kp[c0 + i];
                if (kdst) {
#pragma unroll
                    for (int i = 0; i < kLine; ++i) kdst[c0 + i] = kv[i];
                }
#pragma unroll
                for (int i = 0; i < kLine; ++i) {
                    const int c = c0 + i;
                    const uint32_t w[4] = {kv[i].x, kv[i].y, kv[i].z, kv[i].w};
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const float k0 = bf16_lo(w[t]), k1 = bf16_hi(w[t]);
#pragma unroll
                        for (int r = 0; r < RB; ++r) {
                            acc[r] = __builtin_fmaf(qs[r * D + 8 * c + 2 * t], k0, acc[r]);
                            acc[r] = __builtin_fmaf(qs[r * D + 8 * c + 2 * t + 1], k1, acc[r]);
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const bool seen = valid && r < R && j <= a.new0 + a.s0 + (rz0 + r) / a.rep;
            sc[r] = seen ? bf16_round(bf16_round(acc[r]) * a.scale) : ninf;
        }
    }
    // row max, then sum of exp(s - max) (lanes by butterfly, waves in wave
    // order), then the bf16 weights (:136)
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const float m = wave_max(sc[r]);
        if (lane == 0) wred[wave][r] = m;
    }
    __syncthreads();
    if (tid < RB) {
        float m = wred[0][tid];
#pragma unroll
        for (int w = 1; w < W; ++w) m = fmaxf(m, wred[w][tid]);
        rmax[tid] = m;
    }
    __syncthreads();
    float pw[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        pw[r] = sc[r] == ninf ? 0.0f : att_exp(sc[r] - rmax[r]);
        const float l = wave_sum(pw[r]);
        if (lane == 0) wred[wave][r] = l;
    }
    __syncthreads();
    if (tid < RB) {
        float l = wred[0][tid];
#pragma unroll
        for (int w = 1; w < W; ++w) l = l + wred[w][tid];
        rinv[tid] = 1.0f / l;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RB; ++r) pw[r] = r < R ? bf16_round(pw[r] * rinv[r]) : 0.0f;

    // P.V (:137): wave w over its lanes' positions, value rows in flight
    float acc[RB][E];
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int e = 0; e < E; ++e) acc[r][e] = 0.0f;
    if (wave * 64 < a.L) {
        Raw raw[64];
#pragma unroll
        for (int u = 0; u < 64; ++u) {
            const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)vrow, u);
            const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(vrow >> 32), u);
            const uint16_t *vr = (const uint16_t *)(uintptr_t)(((uint64_t)hi << 32) | lo);
            raw[u] = *gbl((const Raw *)(vr + E * lane));
        }
#pragma unroll
        for (int u = 0; u < 64; ++u) {
            // (positions past the end read the last row with weight 0)
            float v[E];
            if constexpr (E == 1) {
                v[0] = bf16_bits(raw[u]);
            } else if constexpr (E == 2) {
                v[0] = bf16_lo(raw[u]);
                v[1] = bf16_hi(raw[u]);
            } else {
                v[0] = bf16_lo(raw[u].x);
                v[1] = bf16_hi(raw[u].x);
                v[2] = bf16_lo(raw[u].y);
                v[3] = bf16_hi(raw[u].y);
            }
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pw[r]), u));
#pragma unroll
                for (int e = 0; e < E; ++e) acc[r][e] = __builtin_fmaf(w, v[e], acc[r][e]);
            }
        }
    }
    if (wave != 0) {
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int e = 0; e < E; ++e) red[((wave - 1) * RB + r) * D + E * lane + e] = acc[r][e];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        if (r >= R) continue;
        const int s = (rz0 + r) / a.rep, h = kvh * a.rep + (rz0 + r - s * a.rep);
        const size_t row = (size_t)(a.s0 + s) * a.H + h;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int d = E * lane + e;
            float x = acc[r][e];
#pragma unroll
            for (int w = 0; w < W - 1; ++w) x = x + red[(w * RB + r) * D + d];
            uint16_t o = f32_to_bf16(x);
            if (a.gate) {   // :139
                const float g = bf16_bits(a.gate[row * a.gate_stride + d]);
                const float sig = bf16_round(1.0f / (1.0f + att_exp(-g)));
                o = f32_to_bf16(bf16_bits(o) * sig);
            }
            a.out[row * D + d] = o;
        }
    }
}

template <int D, int RB>
int launch_attn(const AttnArgs &a, int nz, hipStream_t st) {
    static std::once_flag once;
    static hipError_t attr_rc = hipSuccess;
    std::call_once(once, [] {
        attr_rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&attn_pv_kernel<D, RB>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)pv_lds_bytes<D, RB>());
    });
    if (attr_rc != hipSuccess) return ECPU_ERR_DEVICE;
    if constexpr (RB * D <= 1024) {
        if (a.L <= kSmallL && env_int("PILM_HIP_ATTN_SMALL", 1) != 0) {
            attn_small_kernel<D, RB><<<dim3((unsigned)a.Hkv, (unsigned)nz), kSmallL, 0, st>>>(a);
            return ECPU_OK;
        }
    }
    attn_scores_kernel<D, RB><<<dim3((unsigned)a.nchunk, (unsigned)a.Hkv, (unsigned)nz), 256, 0, st>>>(a);
    attn_pv_kernel<D, RB><<<dim3((unsigned)a.ngroups, (unsigned)a.Hkv, (unsigned)nz), 256, pv_lds_bytes<D, RB>(), st>>>(a);
    return ECPU_OK;
}

// Query rows per kv head are computed in buckets of 1, 2, 4, 8, 16, 24 or 32
// (24: MTP verify with 5 tokens of a 4-head GQA group, 20 rows).
int row_bucket(int R) {
    return R <= 1 ? 1 : (R <= 2 ? 2 : (R <= 4 ? 4 : (R <= 8 ? 8 : (R <= 16 ? 16 : (R <= 24 ? 24 : 32)))));
}

template <int D>
int launch_attn_rb(int rb, int nz, const AttnArgs &a, hipStream_t st) {
    switch (rb) {
        case 1: return launch_attn<D, 1>(a, nz, st);
        case 2: return launch_attn<D, 2>(a, nz, st);
        case 4: return launch_attn<D, 4>(a, nz, st);
        case 8: return launch_attn<D, 8>(a, nz, st);
        case 16: return launch_attn<D, 16>(a, nz, st);
        case 24: return launch_attn<D, 24>(a, nz, st);
        default: return launch_attn<D, 32>(a, nz, st);
    }
}

}  // namespace

int run_paged_attention(const ekernel_paged_attention_desc_t *d, const uint16_t *q, const uint16_t *k_new,
                        const uint16_t *v_new, uint16_t *k_cache, uint16_t *v_cache, const int32_t *block_ids,
                        const uint16_t *gate, uint16_t *out, hipStream_t st, const char *fn) {
    const int S = (int)d->S, H = (int)d->n_heads, Hkv = (int)d->n_kv_heads, D = (int)d->head_dim;
    const int rep = H / Hkv;
    const int L_total = (int)d->cache_len;
    // query rows per launch: the most tokens whose heads fit kMaxRows rows
    const int per = std::max(1, std::min(S, kMaxRows / rep));
    const int rb_full = row_bucket(per * rep);
    const int Lp_max = (L_total + kChunk - 1) / kChunk * kChunk;
    const int nchunk_max = Lp_max / kChunk;
    const size_t score_floats = ((size_t)Hkv * rb_full * Lp_max * sizeof(uint16_t) + 3) / 4;
    const size_t stat_floats = (size_t)nchunk_max * Hkv * rb_full * 2;
    const size_t part_floats = (size_t)nchunk_max * Hkv * rb_full * D;
    float *P = nullptr;
    int *T = nullptr;
    const size_t pad = 64;   // keep each region 256-byte aligned
    const size_t off_stat = (score_floats + pad - 1) / pad * pad;
    const size_t off_gstat = off_stat + (stat_floats + pad - 1) / pad * pad;
    const size_t off_part = off_gstat + ((size_t)Hkv * rb_full * 2 + pad - 1) / pad * pad;
    int rc = split_scratch(st, off_part + part_floats, 8 * (size_t)Hkv, &P, &T, fn);
    if (rc != ECPU_OK) return rc;

    AttnArgs a;
    a.q = q;
    a.k_new = k_new;
    a.v_new = v_new;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.block_ids = block_ids;
    a.gate = gate;
    a.out = out;
    a.scores = (uint16_t *)P;
    a.stats = P + off_stat;
    a.gstat = P + off_gstat;
    a.part = P + off_part;
    a.tickets = T;
    a.H = H;
    a.Hkv = Hkv;
    a.rep = rep;
    a.new0 = L_total - S;
    a.BS = k_cache ? (int)d->block_size : 1;
    a.NB = k_cache ? (int)d->num_blocks : 1;
    a.gate_stride = (int)d->gate_stride;
    a.scale = (float)(1.0 / std::sqrt((double)D));
    for (int s0 = 0; s0 < S; s0 += per) {
        a.s0 = s0;
        a.S = std::min(per, S - s0);
        const int R = a.S * rep;
        int rb = row_bucket(R);
        a.L = a.new0 + s0 + a.S;
        a.Lp = (a.L + kChunk - 1) / kChunk * kChunk;
        a.nchunk = a.Lp / kChunk;
        // The score pass folds the chunk statistics once beyond 8 chunks (a
        // ticket); below, each P.V wave reads them all.  At most 64 P.V
        // workgroups per kv head keep the final fold short (one workgroup
        // taking two or three chunks in turn measured slower than the fold).
        a.fold_in_pv = a.nchunk <= 8 ? 1 : 0;
        a.cpw = (a.nchunk + 63) / 64;
        a.ngroups = (a.nchunk + a.cpw - 1) / a.cpw;
        a.write_cache = k_cache != nullptr ? 1 : 0;
        // scores keep the first launch's row stride so the regions stay in bounds
        if (rb > rb_full) return fail(ECPU_ERR_DEVICE, "%s: internal row bucket", fn);
        // Query rows in groups on the grid's third dimension, each group
        // rereading the kv head's K and V: more than 8 rows go in groups of 8
        // where the grid is small or the sequence's K and V stay in the 256 MB
        // last-level cache, and groups halve while the grid has fewer than
        // 512 workgroups (one per kv head and group for the one-launch
        // kernel, one per chunk for the two-launch one).  Measured: 8B MTP
        // verify (5 tokens x 4 heads) at 4096 positions 87.7 -> 33.6 us, at
        // 32768 246 -> 161 us; 8B decode at 384 positions 18.0 -> 12.1 us;
        // 1.7B 4-token verify at 4096 41.3 -> 27.1 us.
        int nz = 1;
        const int env_rg = env_int("PILM_HIP_ATTN_ROWGROUPS", 1);   // 0 never, 2 always (groups of 8)
        if (env_rg != 0) {
            const size_t kv_bytes = (size_t)a.L * Hkv * D * 2 * 2;
            const bool one_launch = a.L <= kSmallL;
            const size_t base = one_launch ? (size_t)Hkv : (size_t)a.nchunk * Hkv;
            int g = rb;
            if (rb > 8 && (env_rg == 2 || base < 512 || kv_bytes <= ((size_t)192 << 20))) g = 8;
            if (env_rg != 2)
                while (g > 1 && (size_t)((R + g - 1) / g) * base < 512) g /= 2;
            g = row_bucket(g);
            nz = (R + g - 1) / g;
            rb = g;
        }
        switch (D) {
            case 64: rc = launch_attn_rb<64>(rb, nz, a, st); break;
            case 128: rc = launch_attn_rb<128>(rb, nz, a, st); break;
            default: rc = launch_attn_rb<256>(rb, nz, a, st); break;
        }
        if (rc != ECPU_OK) return fail(ECPU_ERR_DEVICE, "%s: raising the LDS limit of the attention kernel failed", fn);
        rc = check_launch(fn);
        if (rc != ECPU_OK) return rc;
    }
    return ECPU_OK;
}

}  // namespace pilm

using namespace pilm;

namespace {

int check_buf(const void *p, size_t bytes, const char *what, const char *fn) {
    if (!p) return fail(ECPU_ERR_PARAM, "%s: %s is NULL", fn, what);
    return check_device_buffer(p, bytes, what, fn);
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" int ekernel_paged_attention_bf16(const ekernel_paged_attention_desc_t *desc, const uint16_t *q,
                                            const uint16_t *k_new, const uint16_t *v_new, uint16_t *k_cache,
                                            uint16_t *v_cache, const int32_t *block_ids, const uint16_t *gate,
                                            uint16_t *out) {
    static const char *fn = "ekernel_paged_attention_bf16";
    if (!desc) return fail(ECPU_ERR_PARAM, "%s: desc is NULL", fn);
    const size_t S = desc->S, H = desc->n_heads, Hkv = desc->n_kv_heads, D = desc->head_dim;
    if (S == 0) return ECPU_OK;
    if (H == 0 || Hkv == 0 || H % Hkv != 0)
        return fail(ECPU_ERR_PARAM, "%s: n_heads (%zu) must be a positive multiple of n_kv_heads (%zu)", fn, H, Hkv);
    if (H / Hkv > (size_t)kMaxRows)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: more than %d query heads per kv head", fn, kMaxRows);
    if (D != 64 && D != 128 && D != 256) return fail(ECPU_ERR_UNSUPPORTED, "%s: head_dim %zu (64, 128 or 256)", fn, D);
    const size_t L = desc->cache_len;
    if (L < S) return fail(ECPU_ERR_PARAM, "%s: cache_len (%zu) is smaller than S (%zu)", fn, L, S);
    if (L > (size_t)INT_MAX / 2 || S * H * D > (size_t)INT_MAX)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: sequence too long", fn);
    if ((k_cache == nullptr) != (v_cache == nullptr))
        return fail(ECPU_ERR_PARAM, "%s: k_cache and v_cache must both be given or both be NULL", fn);
    int rc;
    if ((rc = check_buf(q, S * H * D * 2, "q", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(k_new, S * Hkv * D * 2, "k_new", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(v_new, S * Hkv * D * 2, "v_new", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(out, S * H * D * 2, "out", fn)) != ECPU_OK) return rc;
    if (!aligned16(q) || !aligned16(k_new) || !aligned16(v_new))
        return fail(ECPU_ERR_PARAM, "%s: q, k_new and v_new must be 16-byte aligned", fn);
    if (k_cache) {
        const size_t BS = desc->block_size, NB = desc->num_blocks, nids = desc->n_block_ids;
        if (BS == 0 || NB == 0) return fail(ECPU_ERR_PARAM, "%s: block_size and num_blocks must be positive", fn);
        if (nids < (L + BS - 1) / BS)
            return fail(ECPU_ERR_PARAM, "%s: %zu block ids cannot hold %zu positions of %zu per block", fn, nids, L, BS);
        if (NB > (size_t)INT_MAX || BS > (size_t)INT_MAX) return fail(ECPU_ERR_UNSUPPORTED, "%s: cache too large", fn);
        const size_t cache_bytes = NB * BS * Hkv * D * 2;
        if ((rc = check_buf(k_cache, cache_bytes, "k_cache", fn)) != ECPU_OK) return rc;
        if ((rc = check_buf(v_cache, cache_bytes, "v_cache", fn)) != ECPU_OK) return rc;
        if ((rc = check_buf(block_ids, nids * 4, "block_ids", fn)) != ECPU_OK) return rc;
        if (!aligned16(k_cache) || !aligned16(v_cache))
            return fail(ECPU_ERR_PARAM, "%s: k_cache and v_cache must be 16-byte aligned", fn);
    } else if (L != S) {
        return fail(ECPU_ERR_PARAM, "%s: without a cache, cache_len (%zu) must equal S (%zu)", fn, L, S);
    }
    if (gate) {
        const size_t gs = desc->gate_stride;
        if (gs < D || gs > (size_t)INT_MAX) return fail(ECPU_ERR_PARAM, "%s: gate_stride %zu is below head_dim", fn, gs);
        if ((rc = check_buf(gate, ((S * H - 1) * gs + D) * 2, "gate", fn)) != ECPU_OK) return rc;
    }
    return run_paged_attention(desc, q, k_new, v_new, k_cache, v_cache, block_ids, gate, out, current_stream(), fn);
}
