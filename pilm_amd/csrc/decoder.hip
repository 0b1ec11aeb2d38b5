// The elementwise and attention steps of one Qwen3 decoder layer on gfx950,
// with the roundings of piLM's torch CPU path (src/models/base/layers.py:101-176,
// src/models/qwen3/attention.py:95-139, src/models/qwen3/model.py:10-127).
//
// piLM runs these steps in torch on the CPU.  Greedy tokens of a random-init
// model sit on bf16 near-ties, so every rounding of that path is kept here:
//   * sums in torch's CPU orders: the reduction of `mean` over a contiguous
//     row (eight-float vectors, four interleaved accumulators, a cascade of
//     16-row levels, then the lanes in order), the softmax's lane reduction
//     (chains j mod 8 folded ((0+4)+(2+6))+((1+5)+(3+7))), the score dot of
//     the bf16 batched product (a halving tree: element i paired with
//     i + D/2, then i + D/4, ...), and its P.V dot (four accumulators on
//     j mod 4, the tail on the first, folded in order);
//   * exp as torch's CPU kernels compute it for softmax, sigmoid and silu
//     (SLEEF's expf_u10, restated below from its published algorithm);
//   * every intermediate tensor rounded to bf16 where torch's is bf16, every
//     fp32 product and sum rounded separately (no contraction), true division
//     and square root.
// The products of two bf16 values are exact in fp32, so an FMA there rounds
// exactly like torch's separate multiply and add.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>

#include "cpu_order.h"
#include "gemv_device.h"
#include "internal.h"

#pragma clang fp contract(off)

namespace pilm {

namespace {

// ---- residual add + GemmaRMSNorm ------------------------------------------
// Row m: h = bf16(x + residual) (or x), residual_out = h, out = norm(h).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t *__restrict__ x,
                                                      const uint16_t *__restrict__ res,
                                                      const uint16_t *__restrict__ w, uint16_t *__restrict__ out,
                                                      uint16_t *__restrict__ res_out, int n, float eps) {
    extern __shared__ float lds[];
    float *xs = lds, *rsh = lds + n;
    const size_t row = (size_t)blockIdx.x * n;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float h = bf(x[row + i]);
        if (res) {
            h = bfr(h + bf(res[row + i]));
            if (res_out) res_out[row + i] = f32_to_bf16(h);
        }
        xs[i] = h;
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const float r = wave_row_rsqrt(xs, n, eps);
        if (threadIdx.x == 0) *rsh = r;
    }
    __syncthreads();
    const float r = *rsh;
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[row + i] = gemma_out(xs[i], r, w[i]);
}

// The same with every load of the row issued at once: thread t owns the
// eight-element chunks t, t + 256, ... (CPT of them; 16-byte loads of x, the
// residual and the weight), so the row costs one memory round trip.  Needs
// n % 8 == 0 and 16-byte aligned rows.  residual and residual_out may be the
// same buffer (each chunk is read before it is written).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

template <int CPT>
__global__ __launch_bounds__(256) void rmsnorm_vec_kernel(const uint16_t *__restrict__ x, const uint16_t *res,
                                                          const uint16_t *__restrict__ w, uint16_t *__restrict__ out,
                                                          uint16_t *res_out, int n, float eps) {
    extern __shared__ float lds[];
    float *xs = lds, *rsh = lds + n;
    const size_t row = (size_t)blockIdx.x * n;
    const int nc = n / 8, t = threadIdx.x;
    u32x4 xv[CPT], rv[CPT], wv[CPT];
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const int c = t + 256 * u;
        if (c < nc) {
            xv[u] = ((const u32x4 *)(x + row))[c];
            if (res) rv[u] = ((const u32x4 *)(res + row))[c];
            wv[u] = ((const u32x4 *)w)[c];
        }
    }
    float h[CPT][8];
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const int c = t + 256 * u;
        if (c < nc) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float a = bf16_lo(xv[u][e]), b = bf16_hi(xv[u][e]);
                if (res) {
                    a = bfr(a + bf16_lo(rv[u][e]));
                    b = bfr(b + bf16_hi(rv[u][e]));
                }
                h[u][2 * e] = a;
                h[u][2 * e + 1] = b;
            }
            if (res && res_out) {
                u32x4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = pack_bf16(h[u][2 * e], h[u][2 * e + 1]);
                ((u32x4 *)(res_out + row))[c] = o;
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) xs[8 * c + e] = h[u][e];
        }
    }
    __syncthreads();
    if (n % 32 == 0) {
        // the block sums of torch's sum of squares by every thread, the
        // cascade and the fold by wave 0 (same bits as wave_row_rsqrt)
        float *bs = lds + n + 4;
        row_sumsq_blocks(xs, n, bs, t, 256);
        __syncthreads();
        if (t < 64) {
            const float r = wave_row_rsqrt_blocks(xs, bs, n, eps);
            if (t == 0) *rsh = r;
        }
    } else if (t < 64) {
        const float r = wave_row_rsqrt(xs, n, eps);
        if (t == 0) *rsh = r;
    }
    __syncthreads();
    const float r = *rsh;
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const int c = t + 256 * u;
        if (c < nc) {
            u32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                o[e] = (uint32_t)gemma_out(h[u][2 * e], r, (uint16_t)(wv[u][e] & 0xFFFFu)) |
                       ((uint32_t)gemma_out(h[u][2 * e + 1], r, (uint16_t)(wv[u][e] >> 16)) << 16);
            ((u32x4 *)(out + row))[c] = o;
        }
    }
}

// ---- rows of several sequences in one launch -------------------------------
// Continuous batching: batch row r belongs to a sequence of nrows[r] rows
// whose cache holds len[r] positions after the call; the row sits at
// position pos[r] and the sequence's block table starts at block_ids +
// tbl[r].  Passed by value as a kernel argument (no device copy, capturable).
constexpr int kMaxBatchRows = 128;
struct BatchRows {
    int32_t pos[kMaxBatchRows];
    int32_t len[kMaxBatchRows];
    int32_t nrows[kMaxBatchRows];
    int32_t tbl[kMaxBatchRows];
};
// The single-sequence form: positions from the descriptor or the state word.
struct OneSeq {};

// ---- q/k GemmaRMSNorm + rope + cache write ---------------------------------
// One wave per (s, head): head < H normalizes q (the first D of the head's 2D
// q_proj outputs) into q_out[s, head, :]; head >= H normalizes k of kv head
// head - H and stores it, with v, into the cache at position pos0 + s.  Rope
// (layers.py:150-195, NeoX halves) on the first rot dims: with c, s the fp32
// tables at the position, (a, b) = (x[f], x[f + rot/2]) becomes
// (a c - b s, a s + b c), each product and sum rounded, then bf16.
template <typename RowsT>
__global__ __launch_bounds__(64) void qk_rope_kernel(
    const uint16_t *__restrict__ qg, const uint16_t *__restrict__ kin, const uint16_t *__restrict__ vin,
    size_t q_stride, size_t kv_stride, const uint16_t *__restrict__ qw, const uint16_t *__restrict__ kw,
    const float *__restrict__ cos_t, const float *__restrict__ sin_t, int max_pos, const int32_t *__restrict__ step,
    int pos0_host, uint16_t *__restrict__ q_out, uint16_t *__restrict__ k_cache, uint16_t *__restrict__ v_cache,
    const int32_t *__restrict__ block_ids, int n_block_ids, int block_size, int num_blocks, int H, int Hkv, int D,
    int rot, float eps, RowsT rows) {
    constexpr bool batched = !std::is_same<RowsT, OneSeq>::value;
    __shared__ float xs[256];
    constexpr int kPer = 4;                  // elements per lane (D <= 256)
    const int s = blockIdx.x, head = blockIdx.y, t = threadIdx.x;
    const bool is_q = head < H;
    const int hk = is_q ? head : head - H;
    const uint16_t *src = is_q ? qg + (size_t)s * q_stride + (size_t)hk * 2 * D : kin + (size_t)s * kv_stride + (size_t)hk * D;
    const uint16_t *nw = is_q ? qw : kw;
    const uint16_t *vsrc = vin + (size_t)s * kv_stride + (size_t)hk * D;
    // every load issued before the arithmetic: the head's values, the norm
    // weight, v; then (once the position is known) the rope table entries and
    // the cache block
    int pos;
    const int32_t *bt = block_ids;
    if constexpr (batched) {
        pos = rows.pos[s];
        bt = block_ids + rows.tbl[s];
    } else {
        pos = (step ? step[0] : pos0_host) + s;
    }
    float xr[kPer];
    uint16_t wr[kPer], vr[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int i = t + 64 * u;
        if (i < D) {
            xr[u] = bf(src[i]);
            wr[u] = nw[i];
            if (!is_q) vr[u] = vsrc[i];
        }
    }
    const int pc = min(max(pos, 0), max_pos - 1);
    const int nf = rot / 2;
    float cr[kPer], sr[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int i = t + 64 * u;
        if (i < rot) {
            const int f = i < nf ? i : i - nf;
            cr[u] = cos_t[(size_t)pc * nf + f];
            sr[u] = sin_t[(size_t)pc * nf + f];
        }
    }
    int blk = 0;
    if (!is_q) blk = min(max(bt[min(max(pos / block_size, 0), n_block_ids - 1)], 0), num_blocks - 1);
#pragma unroll
    for (int u = 0; u < kPer; ++u)
        if (t + 64 * u < D) xs[t + 64 * u] = xr[u];
    __syncthreads();
    const float r = wave_row_rsqrt(xs, D, eps);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kPer; ++u)
        if (t + 64 * u < D) xs[t + 64 * u] = bf(gemma_out(xr[u], r, wr[u]));
    __syncthreads();
    uint16_t *dst;
    if (is_q) {
        dst = q_out + ((size_t)s * H + hk) * D;
    } else {
        const size_t row = (((size_t)blk * block_size + pos % block_size) * Hkv + hk) * D;
        dst = k_cache + row;
#pragma unroll
        for (int u = 0; u < kPer; ++u)
            if (t + 64 * u < D) v_cache[row + t + 64 * u] = vr[u];
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int i = t + 64 * u;
        if (i < D) {
            float o = xs[i];
            if (i < rot) {
                const int f = i < nf ? i : i - nf;
                const float a = xs[f], b = xs[f + nf];
                o = i < nf ? (a * cr[u]) - (b * sr[u]) : (a * sr[u]) + (b * cr[u]);
            }
            dst[i] = f32_to_bf16(o);
        }
    }
}

// ---- attention in torch's CPU order ----------------------------------------
// Workgroup (kv head, query row s, column slice z) computes the rep = H / Hkv
// heads that read this kv head, for head dimensions [z * DS, z * DS + DS).
// The slice of every visible value row (64 bytes each) is copied into LDS by
// DMA at the start, up to vcap positions per pass, so the copy overlaps the
// scores and the softmax.  Scores of the visible positions j <= cache_len -
// S + s go to LDS (bf16 values as fp32) and become softmax weights per head;
// then thread (head, column, chain k) sums its chain of P.V (positions
// j = k mod 4; the tail beyond the last multiple of four on chain 0) from the
// staged rows, and chain 0's thread folds the four chains in order and
// applies the gate.  naive: torch's small product kernel
// (S * cache_len * D < 400) sums both dots in plain order.
constexpr int kDS = 32;        // head dimensions per workgroup (64-byte value rows)

template <int D>
__device__ __forceinline__ float score_dot(const float *qr, const uint32_t (&kv)[D / 2], bool naive) {
    if (naive) {
        float dot = 0.0f;
#pragma unroll
        for (int i = 0; i < D; ++i) dot = dot + qr[i] * (i & 1 ? bf16_hi(kv[i / 2]) : bf16_lo(kv[i / 2]));
        return dot;
    }
    float p[D / 2];
#pragma unroll
    for (int i = 0; i < D / 2; ++i) {
        const int i2 = i + D / 2;
        const float ka = i & 1 ? bf16_hi(kv[i / 2]) : bf16_lo(kv[i / 2]);
        const float kb = i2 & 1 ? bf16_hi(kv[i2 / 2]) : bf16_lo(kv[i2 / 2]);
        p[i] = __builtin_fmaf(qr[i], ka, qr[i2] * kb);
    }
#pragma unroll
    for (int w = D / 4; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; ++i) p[i] = p[i] + p[i + w];
    return p[0];
}

// Block index and offset of position j in a paged cache: shifts when the
// block size is a power of two (the staging loops compute this per 16-byte
// piece, where an integer division would cost more than the copy's issue).
__device__ __forceinline__ void split_pos(int j, int block_size, int &bi, int &off) {
    if ((block_size & (block_size - 1)) == 0) {
        bi = j >> __builtin_ctz(block_size);
        off = j & (block_size - 1);
    } else {
        bi = j / block_size;
        off = j - bi * block_size;
    }
}

// LDS DMA of the cache rows [j0, j0 + nrows) (nrows >= 1): PPR 16-byte
// pieces per row from base (a kv head's first column of the slice; rows
// row_elems apart), staging row r at dst + r * PPR * 8 elements; SWZ stores
// piece c of row r in slot c ^ (r mod PPR).  Whole instructions of every
// wave (pieces past the rows repeat the last row), four pieces per thread per
// round so that the round's block table reads share one wait.
template <int PPR, int NT, bool SWZ>
__device__ __forceinline__ void stage_rows(const uint16_t *base, uint32_t row_elems, const int *bids, int n_block_ids,
                                           int block_size, int j0, int nrows, uint16_t *dst, int t) {
    const int wave = t >> 6;
    const int pieces = ((nrows * PPR + NT - 1) / NT) * NT;
    for (int b = 0; b < pieces; b += 4 * NT) {
        size_t off[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int idx = b + u * NT + t;
            const int r = min(idx / PPR, nrows - 1);
            const int slot = idx % PPR;
            const int c = SWZ ? (slot ^ (r & (PPR - 1))) : slot;
            int bi, o;
            split_pos(j0 + r, block_size, bi, o);
            const uint32_t row = (uint32_t)bids[min(bi, n_block_ids - 1)] * (uint32_t)block_size + (uint32_t)o;
            off[u] = (size_t)row * row_elems + 8 * c;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (b + u * NT < pieces)
                __builtin_amdgcn_global_load_lds((const void *)(base + off[u]),
                                                 (lds_void *)(dst + (size_t)(b + u * NT + wave * 64) * 8), 16, 0, 0);
    }
}

// Sum of x[0 .. vis) in torch's order for a row of cache_len positions (every
// lane of the wave gets it): eight chains j = c mod 8, each in order, folded
// as ((0+4) + (2+6)) + ((1+5) + (3+7)); one plain chain below eight.
__device__ __forceinline__ float exp_sum(const float *x, int vis, int cache_len, int lane) {
    float sum = 0.0f;
    if (cache_len >= 8) {
        // lane c < 8: chain c = positions j = c mod 8, in order from x[c]
        float a = 0.0f;
        if (lane < 8) {
            a = lane < vis ? x[lane] : 0.0f;
            int j = lane + 8;
            for (; j + 56 < vis; j += 64) {
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = x[j + 8 * u];
#pragma unroll
                for (int u = 0; u < 8; ++u) a = a + v[u];
            }
            for (; j < vis; j += 8) a = a + x[j];
        }
        float l[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) l[q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), q));
        sum = ((l[0] + l[4]) + (l[2] + l[6])) + ((l[1] + l[5]) + (l[3] + l[7]));
    } else {
        for (int j = 0; j < vis; ++j) sum = sum + x[j];
    }
    return sum;
}

// exp_sum over values stored by chain: x[j] at xc[(j mod 8) * cs + j / 8]
// (cs a multiple of four, xc 16-byte aligned), so that lane c reads its
// chain four values at a time; the same order of additions.
__device__ __forceinline__ float exp_sum_chains(const float *xc, int cs, int vis, int cache_len, int lane) {
    float sum = 0.0f;
    if (cache_len >= 8) {
        float a = 0.0f;
        if (lane < 8) {
            const float *x = xc + lane * cs;
            const int n = (vis - lane + 7) / 8;          // positions lane + 8 i below vis
            if (n > 0) a = x[0];
            int i = 1;
            for (; i < min(n, 4); ++i) a = a + x[i];
            for (; i + 16 <= n; i += 16) {
                float4 v[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) v[u] = *(const float4 *)(x + i + 4 * u);
#pragma unroll
                for (int u = 0; u < 4; ++u) a = (((a + v[u].x) + v[u].y) + v[u].z) + v[u].w;
            }
            for (; i + 4 <= n; i += 4) {
                const float4 v = *(const float4 *)(x + i);
                a = (((a + v.x) + v.y) + v.z) + v.w;
            }
            for (; i < n; ++i) a = a + x[i];
        }
        float l[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) l[q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), q));
        sum = ((l[0] + l[4]) + (l[2] + l[6])) + ((l[1] + l[5]) + (l[3] + l[7]));
    } else {
        for (int j = 0; j < vis; ++j) sum = sum + xc[(j & 7) * cs + (j >> 3)];
    }
    return sum;
}

// One wave turns the bf16 scores x[0 .. vis) of a row (cache_len positions
// long with the masked ones) into bf16 softmax weights in place: max, exp,
// the sum in torch's order (eight chains j = c mod 8 folded as ((0+4) +
// (2+6)) + ((1+5) + (3+7)); one plain chain below eight positions), then
// x * (1 / sum) rounded to bf16.
__device__ __forceinline__ void softmax_weights(float *x, int vis, int cache_len, int lane) {
    float mx = -__builtin_inff();
    for (int j = lane; j < vis; j += 64) mx = fmaxf(mx, x[j]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    for (int j = lane; j < vis; j += 64) x[j] = sleef_expf(x[j] - mx);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float inv = __fdiv_rn(1.0f, exp_sum(x, vis, cache_len, lane));
    for (int j = lane; j < vis; j += 64) x[j] = bfr(x[j] * inv);
}

template <int D>
__device__ __forceinline__ void load_krow(const uint16_t *kr, uint32_t (&kv)[D / 2]) {
#pragma unroll
    for (int i = 0; i < D / 8; ++i) {
        const u32x4 c = ((const u32x4 *)kr)[i];
        kv[4 * i] = c[0];
        kv[4 * i + 1] = c[1];
        kv[4 * i + 2] = c[2];
        kv[4 * i + 3] = c[3];
    }
}

template <int D, typename RowsT>
__global__ __launch_bounds__(256) void attn_exact_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k_cache, const uint16_t *__restrict__ v_cache,
    const int32_t *__restrict__ block_ids, int n_block_ids, int num_blocks, int block_size,
    const uint16_t *__restrict__ gate, size_t gate_row_stride, size_t gate_head_stride,
    const int32_t *__restrict__ step, int cache_len_host, int S_call, int H, int Hkv, int max_len, int vcap,
    float scale, uint16_t *__restrict__ out, RowsT rows) {
    constexpr bool batched = !std::is_same<RowsT, OneSeq>::value;
    extern __shared__ float lds[];
    const int kh = blockIdx.x, s = blockIdx.y, z = blockIdx.z, t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63;
    const int rep = H / Hkv;
    // this row's sequence: its rows (S), its cached length and the row's
    // visible positions 0 .. vis-1
    int S, cache_len, vis;
    if constexpr (batched) {
        S = max(rows.nrows[s], 1);
        cache_len = min(max(rows.len[s], S), max_len);
        vis = min(max(rows.pos[s], cache_len - S), cache_len - 1) + 1;
        block_ids += rows.tbl[s];
    } else {
        S = S_call;
        cache_len = step ? step[1] : cache_len_host;
        cache_len = min(max(cache_len, S), max_len);
        vis = cache_len - S + s + 1;
    }
    const bool naive = (long long)S * cache_len * D < 400;
    const int scs = (max_len + 3) & ~3;                        // score row stride (16-byte rows)
    float *qs = lds;                                           // [rep][D]
    float *sc = qs + rep * D;                                  // [rep][scs]
    float *part = sc + (size_t)rep * scs;                      // [rep][kDS][4] chain sums
    int *bids = (int *)(part + rep * kDS * 4);                 // [n_block_ids]
    uint16_t *vs = (uint16_t *)(bids + ((n_block_ids + 3) & ~3));   // [vcap][kDS]
    const int d0 = z * kDS;
    for (int i = t; i < n_block_ids; i += blockDim.x) bids[i] = min(max(block_ids[i], 0), num_blocks - 1);
    for (int i = t; i < rep * D; i += blockDim.x) {
        const int r = i / D, d = i % D;
        qs[i] = bf(q[((size_t)s * H + kh * rep + r) * D + d]);
    }
    // the gate values of this thread's outputs (P.V pass it, chain 0), fetched
    // with q rather than after the sums; passes beyond kGatePre load theirs late
    constexpr int kGatePre = 4;
    const int nthr = rep * kDS * 4;
    float gpre[kGatePre];
#pragma unroll
    for (int it = 0; it < kGatePre; ++it) {
        const int i = it * (int)blockDim.x + t;
        gpre[it] = 0.0f;
        if (gate && i < nthr && (i & 3) == 0) {
            const int h = kh * rep + i / (kDS * 4), dd = d0 + (i / 4) % kDS;
            gpre[it] = bf(gate[(size_t)s * gate_row_stride + (size_t)h * gate_head_stride + dd]);
        }
    }
    __syncthreads();

    auto row_of = [&](int j) -> size_t {
        int bi, off;
        split_pos(j, block_size, bi, off);
        const uint32_t row = (uint32_t)bids[min(bi, n_block_ids - 1)] * (uint32_t)block_size + (uint32_t)off;
        return (size_t)row * (uint32_t)(Hkv * D) + (size_t)kh * D;
    };
    // value rows [j0, j0 + vcap) of this slice into vs: 16 bytes per lane,
    // four lanes per row; rows past the visible ones repeat the last visible
    // row (never read).
    auto stage_v = [&](int j0) {
        stage_rows<kDS / 8, 256, false>(v_cache + (size_t)kh * D + d0, (uint32_t)(Hkv * D), bids, n_block_ids,
                                        block_size, j0, min(vcap, vis - j0), vs, t);
    };
    stage_v(0);

    // scores: two positions per thread in flight (one for 256-wide heads)
    constexpr int kPer = D <= 128 ? 2 : 1;
    for (int j = t; j < vis; j += kPer * blockDim.x) {
        const int j2 = kPer == 2 ? j + blockDim.x : vis;
        uint32_t ka[D / 2], kb[D / 2];
        load_krow<D>(k_cache + row_of(j), ka);
        if (j2 < vis) load_krow<D>(k_cache + row_of(j2), kb);
        for (int r = 0; r < rep; ++r) {
            const float *qr = qs + r * D;
            sc[(size_t)r * scs + j] = bfr(bfr(score_dot<D>(qr, ka, naive)) * scale);
            if (j2 < vis) sc[(size_t)r * scs + j2] = bfr(bfr(score_dot<D>(qr, kb, naive)) * scale);
        }
    }
    __syncthreads();

    // softmax per head: wave r (looping when rep exceeds the wave count)
    for (int r = wave; r < rep; r += blockDim.x / 64) softmax_weights(sc + (size_t)r * scs, vis, cache_len, lane);

    // P.V: thread (r, column c, chain k) over the staged value rows
    const int main_len = naive ? 0 : (cache_len / 4) * 4;
    for (int base = 0; base < nthr; base += blockDim.x) {
        const int i = base + t;
        const bool active = i < nthr;
        const int r = active ? i / (kDS * 4) : 0, c = (i / 4) % kDS, k = i & 3;
        const float *w = sc + (size_t)r * scs;
        float acc = 0.0f;
        for (int j0 = 0; j0 < vis; j0 += vcap) {
            if (j0 > 0 || base > 0) {
                __syncthreads();          // the previous rows have been read
                stage_v(j0);
            }
            wait_vmcnt<0>();
            __syncthreads();              // every wave's copies (and the weights) are in
            const int j1 = min(vis, j0 + vcap);
            if (active) {
                if (naive) {
                    if (k == 0)
                        for (int j = j0; j < j1; ++j) acc = __builtin_fmaf(w[j], bf(vs[(j - j0) * kDS + c]), acc);
                } else {
                    // chain k: positions j = k mod 4 below main_len; chain 0 also takes the tail
                    int j = j0 + ((k - j0) & 3);
                    const int jm = min(j1, main_len);
                    for (; j + 12 < jm; j += 16) {
                        float wv[4], vv[4];
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            wv[u] = w[j + 4 * u];
                            vv[u] = bf(vs[(j + 4 * u - j0) * kDS + c]);
                        }
#pragma unroll
                        for (int u = 0; u < 4; ++u) acc = __builtin_fmaf(wv[u], vv[u], acc);
                    }
                    for (; j < jm; j += 4) acc = __builtin_fmaf(w[j], bf(vs[(j - j0) * kDS + c]), acc);
                    if (k == 0)
                        for (j = max(j0, main_len); j < j1; ++j)
                            acc = __builtin_fmaf(w[j], bf(vs[(j - j0) * kDS + c]), acc);
                }
            }
        }
        if (active) part[i - base] = acc;
        __syncthreads();
        if (active && k == 0) {
            const float *pp = part + (i - base);
            float o = naive ? pp[0] : ((pp[0] + pp[1]) + pp[2]) + pp[3];
            o = bfr(o);
            const int h = kh * rep + r, d = d0 + c;
            if (gate) {
                const int it = base / (int)blockDim.x;
                const float g = it == 0 ? gpre[0] : it == 1 ? gpre[1] : it == 2 ? gpre[2] : it == 3 ? gpre[3]
                              : bf(gate[(size_t)s * gate_row_stride + (size_t)h * gate_head_stride + d]);
                o = o * bfr(__fdiv_rn(1.0f, 1.0f + sleef_expf(-g)));
            }
            out[((size_t)s * H + h) * D + d] = f32_to_bf16(o);
        }
    }
}

// ---- attention over several rows of one sequence ----------------------------
// Continuous batching: a workgroup serves one kv head for a tile of
// consecutive rows of one sequence (rows x rep <= kTileVecs (row, q head)
// vectors), so each key row is loaded once per tile and each score is
// computed once, over the full head width.  Every vector gets exactly what
// attn_exact_kernel computes for its row: the same score order and roundings,
// softmax_weights, the same four P.V chains over the positions the row sees
// (j = k mod 4 below the last multiple of four of cache_len, the tail on
// chain 0), the fold ((p0 + p1) + p2) + p3 and the gate.
// Threads: scores by (position, vector parity); P.V by (vector group g,
// column pair, chain k), the four chains of a column pair in adjacent lanes.
constexpr int kTileVecs = 16;
constexpr int kTileThreads = 512;

struct BatchTiles {
    int32_t tile[kMaxBatchRows];       // first batch row | rows << 16
};

template <int D, int NV>
__global__ __launch_bounds__(kTileThreads) void attn_tile_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k_cache, const uint16_t *__restrict__ v_cache,
    const int32_t *__restrict__ block_ids, int n_block_ids, int num_blocks, int block_size,
    const uint16_t *__restrict__ gate, size_t gate_row_stride, size_t gate_head_stride, int H, int Hkv,
    int max_len, int vecs, int scs, int vcap, float scale, uint16_t *__restrict__ out, BatchRows rows,
    BatchTiles tiles) {
    constexpr int CP = D / 2;                        // column pairs
    constexpr int G = kTileThreads / (4 * CP);       // vector groups of the P.V pass
    static_assert(NV >= 1 && NV * G <= kTileVecs, "vectors per P.V thread");
    constexpr int QS = D + 4;                        // q row stride: the vectors on different banks
    constexpr int PPR = D / 8;                       // 16-byte pieces per value row
    extern __shared__ float lds[];
    const int kh = blockIdx.x, t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int rep = H / Hkv;
    const int row0 = tiles.tile[blockIdx.y] & 0xFFFF, nr = tiles.tile[blockIdx.y] >> 16;
    const int RR = nr * rep;
    const int S = max(rows.nrows[row0], 1);
    const int cache_len = min(max(rows.len[row0], S), max_len);
    auto vis_of = [&](int rr) {                      // visible positions of vector rr's row
        return min(max(rows.pos[row0 + rr / rep], cache_len - S), cache_len - 1) + 1;
    };
    const int vis_min = vis_of(0), vis_max = vis_of(RR - 1);
    const bool naive = (long long)S * cache_len * D < 400;
    const int main_len = naive ? 0 : (cache_len / 4) * 4;
    block_ids += rows.tbl[row0];
    // P.V thread: vectors g + n G (n < NV; the ones past RR compute on a
    // clamped row and are dropped), columns 2 cp, 2 cp + 1, chain k.  Its
    // gate values are fetched now, not after the sums.
    const int k = t & 3, cp = (t >> 2) % CP, g = t / (4 * CP);
    float gv[NV][2];
#pragma unroll
    for (int n = 0; n < NV; ++n) {
        const int rr = g + n * G;
        gv[n][0] = gv[n][1] = 0.0f;
        if (gate && k == 0 && rr < RR) {
            const uint16_t *gp = gate + (size_t)(row0 + rr / rep) * gate_row_stride +
                                 (size_t)(kh * rep + rr % rep) * gate_head_stride + 2 * cp;
            gv[n][0] = bf(gp[0]);
            gv[n][1] = bf(gp[1]);
        }
    }
    float *qs = lds;                                             // [vecs][QS]
    float *sc = qs + (size_t)vecs * QS;                          // [vecs][scs]
    int *bids = (int *)(sc + (size_t)vecs * scs);                // [n_block_ids]
    uint16_t *vs = (uint16_t *)(bids + ((n_block_ids + 3) & ~3));   // [vcap][D]
    for (int i = t; i < n_block_ids; i += kTileThreads) bids[i] = min(max(block_ids[i], 0), num_blocks - 1);
    for (int i = t; i < RR * D; i += kTileThreads) {
        const int rr = i / D, d = i % D;
        qs[rr * QS + d] = bf(q[((size_t)(row0 + rr / rep) * H + kh * rep + rr % rep) * D + d]);
    }
    __syncthreads();

    auto row_of = [&](int j) -> size_t {
        int bi, off;
        split_pos(j, block_size, bi, off);
        const uint32_t row = (uint32_t)bids[min(bi, n_block_ids - 1)] * (uint32_t)block_size + (uint32_t)off;
        return (size_t)row * (uint32_t)(Hkv * D) + (size_t)kh * D;
    };
    // value rows [j0, j0 + vcap) into vs, 16 bytes per lane; whole
    // instructions of every wave, pieces past the rows repeat the last row
    auto stage_v = [&](int j0) {
        stage_rows<PPR, kTileThreads, false>(v_cache + (size_t)kh * D, (uint32_t)(Hkv * D), bids, n_block_ids,
                                             block_size, j0, min(vcap, vis_max - j0), vs, t);
    };
    stage_v(0);

    // scores: thread (position j, vector parity); the key row stays in registers
    for (int j = t % 256; j < vis_max; j += 256) {
        uint32_t ka[D / 2];
        load_krow<D>(k_cache + row_of(j), ka);
        for (int rr = t / 256; rr < RR; rr += kTileThreads / 256)
            if (j < vis_of(rr)) sc[(size_t)rr * scs + j] = bfr(bfr(score_dot<D>(qs + rr * QS, ka, naive)) * scale);
    }
    __syncthreads();
    for (int rr = wave; rr < RR; rr += kTileThreads / 64) softmax_weights(sc + (size_t)rr * scs, vis_of(rr), cache_len, lane);

    // P.V
    int visv[NV], wo[NV];
    float acc[NV][2];
#pragma unroll
    for (int n = 0; n < NV; ++n) {
        const int rr = g + n * G;
        visv[n] = rr < RR ? vis_of(rr) : 0;
        wo[n] = min(rr, RR - 1) * scs;
        acc[n][0] = acc[n][1] = 0.0f;
    }
    const uint32_t *vw = (const uint32_t *)vs;
    for (int j0 = 0; j0 < vis_max; j0 += vcap) {
        if (j0 > 0) {
            __syncthreads();              // every wave is done with the previous rows
            stage_v(j0);
        }
        wait_vmcnt<0>();
        __syncthreads();                  // every wave's copies (and the weights) are in
        const int j1 = min(vis_max, j0 + vcap);
        // every vector of the tile sees j: no condition
        auto step_all = [&](int j) {
            const uint32_t vp = vw[(j - j0) * CP + cp];
            const float v0 = bf16_lo(vp), v1 = bf16_hi(vp);
#pragma unroll
            for (int n = 0; n < NV; ++n) {
                const float w = sc[wo[n] + j];
                acc[n][0] = __builtin_fmaf(w, v0, acc[n][0]);
                acc[n][1] = __builtin_fmaf(w, v1, acc[n][1]);
            }
        };
        // only the vectors whose row sees j take it
        auto step_masked = [&](int j) {
            const uint32_t vp = vw[(j - j0) * CP + cp];
            const float v0 = bf16_lo(vp), v1 = bf16_hi(vp);
#pragma unroll
            for (int n = 0; n < NV; ++n) {
                const float w = sc[wo[n] + j];
                const bool on = j < visv[n];
                acc[n][0] = on ? __builtin_fmaf(w, v0, acc[n][0]) : acc[n][0];
                acc[n][1] = on ? __builtin_fmaf(w, v1, acc[n][1]) : acc[n][1];
            }
        };
        if (naive) {
            if (k == 0)
                for (int j = j0; j < j1; ++j) step_masked(j);
        } else {
            int j = j0 + ((k - j0) & 3);
            const int jm = min(j1, main_len);
            const int ja = min(jm, vis_min);
#pragma unroll 2
            for (; j < ja; j += 4) step_all(j);
            for (; j < jm; j += 4) step_masked(j);
            if (k == 0)
                for (j = max(j0, main_len); j < j1; ++j) step_masked(j);
        }
    }

    // fold the four chains of each column (adjacent lanes), gate, store
    const int lb = lane & ~3;
#pragma unroll
    for (int n = 0; n < NV; ++n) {
        const int rr = g + n * G;
        if (rr >= RR) break;
        float o[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const float a0 = acc[n][c];
            const float a1 = __shfl(a0, lb + 1), a2 = __shfl(a0, lb + 2), a3 = __shfl(a0, lb + 3);
            o[c] = bfr(naive ? a0 : ((a0 + a1) + a2) + a3);
        }
        if (k == 0) {
            const int row = row0 + rr / rep, h = kh * rep + rr % rep, d = 2 * cp;
            if (gate) {
#pragma unroll
                for (int c = 0; c < 2; ++c) o[c] = o[c] * bfr(__fdiv_rn(1.0f, 1.0f + sleef_expf(-gv[n][c])));
            }
            *(uint32_t *)(out + ((size_t)row * H + h) * D + d) =
                (uint32_t)f32_to_bf16(o[0]) | ((uint32_t)f32_to_bf16(o[1]) << 16);
        }
    }
}

// ---- one decode row: q/k norm + rope + cache write + attention ---------------
// The steps of qk_rope_kernel and attn_exact_kernel for S = 1 in one launch.
// A 512-thread workgroup serves HPW of the rep q heads that read one kv head
// (grid: kv heads x rep / HPW): waves 0 .. HPW-1 normalize and rotate those q
// heads, wave HPW the k head (the first workgroup of the kv head also writes
// the k and v rows into the cache).  Key rows come by DMA into LDS, their
// 16-byte chunks XOR-swizzled, the new position's from registers; scores run
// one position per thread.  The value rows follow into the same LDS, and
// thread (chain k, column c), c fastest, sums P.V for the workgroup's heads,
// so a wave reads one value row contiguously and each weight by broadcast.
// Every sum keeps the order of the two-kernel path above.
constexpr int kDecodeThreads = 512;

// Workgroup barrier for LDS traffic only: this wave's LDS operations are
// complete, its global loads and LDS copies may still be in flight.
__device__ __forceinline__ void lds_only_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Largest value of a wave (every lane gets it) through DPP row shifts and
// broadcasts instead of LDS-routed shuffles: max is exact in any order.
__device__ __forceinline__ float wave_max_dpp(float v) {
    const int ninf = __float_as_int(-__builtin_inff());
    auto step = [&](int w) { v = fmaxf(v, __int_as_float(w)); };
    step(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x111, 0xF, 0xF, false));   // row_shr:1
    step(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x112, 0xF, 0xF, false));   // row_shr:2
    step(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x114, 0xF, 0xF, false));   // row_shr:4
    step(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x118, 0xF, 0xF, false));   // row_shr:8
    step(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x142, 0xA, 0xF, false));   // row_bcast:15
    step(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x143, 0xC, 0xF, false));   // row_bcast:31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

template <int D, int REP, int HPW>
__global__ __launch_bounds__(kDecodeThreads) void decode_attn_kernel(
    const uint16_t *__restrict__ qg, const uint16_t *__restrict__ kin, const uint16_t *__restrict__ vin,
    const uint16_t *__restrict__ qw, const uint16_t *__restrict__ kw, const float *__restrict__ cos_t,
    const float *__restrict__ sin_t, int max_pos, const int32_t *__restrict__ step, int pos0_host,
    uint16_t *__restrict__ k_cache, uint16_t *__restrict__ v_cache, const int32_t *__restrict__ block_ids,
    int n_block_ids, int block_size, int num_blocks, int H, int Hkv, int rot, float eps, int max_len, int vcap,
    float scale, uint16_t *__restrict__ out) {
    constexpr int kPer = D / 64;          // elements per lane of one head
    constexpr int nthreads = kDecodeThreads;
    constexpr int rep = REP;              // q heads per kv head (H / Hkv)
    constexpr int hpw = HPW;              // of them, heads of this workgroup: h0 .. h0 + hpw - 1
    static_assert(REP % HPW == 0, "heads per workgroup divide the heads per kv head");
    extern __shared__ float lds[];
    const int kh = blockIdx.x, t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int h0 = kh * rep + blockIdx.y * hpw;
    const bool writer = blockIdx.y == 0;  // the workgroup that stores the new cache rows
    const int scs = (max_len + 3) & ~3;
    float *xn = lds;                                           // [hpw + 1][D] normalized heads
    float *qs = xn + (hpw + 1) * D;                            // [hpw][D] roped q
    float *sc = qs + hpw * D;                                  // [hpw][scs]
    float *part = sc + (size_t)hpw * scs;                      // [hpw][4][D] chain sums
    // one row's exps / weights by chain (the one-pass path: <= nthreads positions)
    constexpr int kC8 = (nthreads / 8 + 3) & ~3, kC4 = (nthreads / 4 + 3) & ~3;   // chain strides
    float *cm = part + hpw * 4 * D;                            // [nthreads + 32]
    int *bids = (int *)(cm + nthreads + 32);                   // [n_block_ids]
    uint16_t *vs = (uint16_t *)(bids + ((n_block_ids + 3) & ~3));   // [vcap][D]

    const int pos = step ? step[0] : pos0_host;
    int cache_len = step ? step[1] : pos0_host + 1;
    cache_len = min(max(cache_len, 1), max_len);
    const int vis = cache_len;
    const bool naive = (long long)cache_len * D < 400;
    const bool pos_ok = pos >= 0 && pos < max_len;
    for (int i = t; i < n_block_ids; i += nthreads) bids[i] = min(max(block_ids[i], 0), num_blocks - 1);

    // the head this wave normalizes: q head h0 + wave, or the k head
    const bool head_wave = wave <= hpw;
    const bool is_k = wave == hpw;
    float xr[kPer];
    uint16_t wr[kPer], vr[kPer], kb[kPer];
    if (head_wave) {
        const uint16_t *src = is_k ? kin + (size_t)kh * D : qg + (size_t)(h0 + wave) * 2 * D;
        const uint16_t *nw = is_k ? kw : qw;
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            xr[u] = bf(src[lane + 64 * u]);
            wr[u] = nw[lane + 64 * u];
            if (is_k) vr[u] = vin[(size_t)kh * D + lane + 64 * u];
        }
    }
    const int pc = min(max(pos, 0), max_pos - 1);
    const int nf = rot / 2;
    float cr[kPer], sr[kPer];
    if (head_wave) {
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int i = lane + 64 * u;
            if (i < rot) {
                const int f = i < nf ? i : i - nf;
                cr[u] = cos_t[(size_t)pc * nf + f];
                sr[u] = sin_t[(size_t)pc * nf + f];
            }
        }
    }
    // the gate values of the outputs this thread folds: (head r, column c) for
    // r * D + c = t + nthreads * it
    constexpr int kGatePre = 2;
    float gpre[kGatePre];
#pragma unroll
    for (int it = 0; it < kGatePre; ++it) {
        const int o = t + nthreads * it;
        gpre[it] = o < hpw * D ? bf(qg[(size_t)(h0 + o / D) * 2 * D + D + o % D]) : 0.0f;
    }
    if (head_wave) {
#pragma unroll
        for (int u = 0; u < kPer; ++u) xn[wave * D + lane + 64 * u] = xr[u];
    }
    __syncthreads();                      // block ids and the raw heads are in

    auto row_of = [&](int j) -> size_t {
        int bi, off;
        split_pos(j, block_size, bi, off);
        const uint32_t row = (uint32_t)bids[min(bi, n_block_ids - 1)] * (uint32_t)block_size + (uint32_t)off;
        return (size_t)row * (uint32_t)(Hkv * D) + (size_t)kh * D;
    };
    // rows [j0, j0 + vcap) of a cache into the staging region: 16 bytes per
    // lane, D / 8 lanes per row, one DMA instruction per 64 pieces; rows past
    // the visible ones repeat the last visible row.  Key rows are stored with
    // their 16-byte chunks XOR-swizzled by the row index (chunk u of row j at
    // slot u ^ (j mod D/8)), so that one thread per row reads them from LDS
    // without bank conflicts; value rows are stored plainly.
    constexpr int per_row = D / 8;
    auto stage = [&](const uint16_t *cache, int j0, bool swizzle) {
        if (swizzle)
            stage_rows<per_row, nthreads, true>(cache + (size_t)kh * D, (uint32_t)(Hkv * D), bids, n_block_ids,
                                                block_size, j0, min(vcap, vis - j0), vs, t);
        else
            stage_rows<per_row, nthreads, false>(cache + (size_t)kh * D, (uint32_t)(Hkv * D), bids, n_block_ids,
                                                 block_size, j0, min(vcap, vis - j0), vs, t);
    };
    stage(k_cache, 0, true);

    if (head_wave) {
        const float r = wave_row_rsqrt(xn + wave * D, D, eps);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int u = 0; u < kPer; ++u) xn[wave * D + lane + 64 * u] = bf(gemma_out(xr[u], r, wr[u]));
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const float *x = xn + wave * D;
        float *dst = qs + wave * D;       // roped q
        const size_t crow = (is_k && pos_ok && writer) ? row_of(pos) : 0;
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int i = lane + 64 * u;
            float o = x[i];
            if (i < rot) {
                const int f = i < nf ? i : i - nf;
                const float a = x[f], b = x[f + nf];
                o = i < nf ? (a * cr[u]) - (b * sr[u]) : (a * sr[u]) + (b * cr[u]);
            }
            const uint16_t ob = f32_to_bf16(o);
            if (!is_k) dst[i] = bf(ob);
            kb[u] = ob;
            if (is_k && pos_ok && writer) {
                k_cache[crow + i] = ob;
                v_cache[crow + i] = vr[u];
            }
        }
    }

    // scores from the staged key rows, one position per thread; the new
    // position's row is written into the staging from registers (the copy the
    // DMA brought may predate the cache write).  When every position is one
    // thread's and one staging pass holds them, each thread first copies its
    // key row to registers and the value rows' DMA into the same region
    // starts at once, under the scores (an LDS-only barrier after them; the
    // softmax's LDS writes then wait for the DMA).
    // One q head per workgroup and one position per thread: each thread
    // loads its share of the value rows into registers as soon as the key
    // rows are out of the staging (plain loads, so the LDS traffic of the
    // scores and the softmax does not wait for them, as it would for LDS
    // copies), every wave computes scores and the softmax (max over DPP and
    // the waves' maxima, exp, the chain sums on wave 0, the weights), and
    // the value rows go into the staging before the P.V pass.
    constexpr int kWaves = nthreads / 64;
    const bool split_v = HPW == 1 && vis <= nthreads && vis <= vcap;
    const bool early_v = !split_v && vis <= nthreads && vis <= vcap;
    if (split_v) {
        wait_vmcnt<0>();
        __syncthreads();                  // the key rows (and the roped q and k) are in
        if (is_k && pos >= 0 && pos < vis) {
#pragma unroll
            for (int u = 0; u < kPer; ++u) {
                const int i = lane + 64 * u;
                vs[(size_t)pos * D + 8 * ((i / 8) ^ (pos & (per_row - 1))) + i % 8] = kb[u];
            }
        }
        __syncthreads();
        uint32_t ka[D / 2];
        if (t < vis) {
            const uint16_t *row = vs + (size_t)t * D;
#pragma unroll
            for (int u = 0; u < per_row; ++u) {
                const u32x4 c = *(const u32x4 *)(row + 8 * (u ^ (t & (per_row - 1))));
                ka[4 * u] = c[0];
                ka[4 * u + 1] = c[1];
                ka[4 * u + 2] = c[2];
                ka[4 * u + 3] = c[3];
            }
        }
        // piece u of this thread: value row t / per_row + u * nthreads / per_row,
        // chunk t mod per_row; the block table reads first, then the loads
        uint32_t vrow[per_row];
#pragma unroll
        for (int u = 0; u < per_row; ++u) {
            int bi, o;
            split_pos(min(t / per_row + u * (nthreads / per_row), vis - 1), block_size, bi, o);
            vrow[u] = (uint32_t)bids[min(bi, n_block_ids - 1)] * (uint32_t)block_size + (uint32_t)o;
        }
        const uint16_t *vbase = v_cache + (size_t)kh * D + 8 * (t % per_row);
        u32x4 vp[per_row];
#pragma unroll
        for (int u = 0; u < per_row; ++u)
            if (t / per_row + u * (nthreads / per_row) < vis)
                vp[u] = *(const u32x4 *)(vbase + (size_t)vrow[u] * (uint32_t)(Hkv * D));
        float *red = part;                // [kWaves] the waves' maxima, then 1 / sum
        float e = -__builtin_inff();
        if (t < vis) e = bfr(bfr(score_dot<D>(qs, ka, naive)) * scale);
        const float m = wave_max_dpp(e);
        if (lane == 0) red[wave] = m;
        lds_only_barrier();               // every wave's maximum (and every key row read)
        float mx = red[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, red[w]);
        // the exps by sum chain (position j at cm[(j mod 8) c8 + j / 8]), then
        // the weights by P.V chain (cm[(j mod 4) c4 + j / 4]) besides sc[j]
        constexpr int c8 = kC8, c4 = kC4;
        if (t < vis) {
            e = sleef_expf(e - mx);
            cm[(t & 7) * c8 + (t >> 3)] = e;
        }
        lds_only_barrier();
        if (wave == 0) {
            const float inv = __fdiv_rn(1.0f, exp_sum_chains(cm, c8, vis, cache_len, lane));
            if (lane == 0) red[kWaves] = inv;
        }
        lds_only_barrier();
        if (t < vis) {
            const float w = bfr(e * red[kWaves]);
            sc[t] = w;
            cm[(t & 3) * c4 + (t >> 2)] = w;
        }
#pragma unroll
        for (int u = 0; u < per_row; ++u) {
            const int r = t / per_row + u * (nthreads / per_row);
            if (r < vis) *(u32x4 *)(vs + (size_t)r * D + 8 * (t % per_row)) = vp[u];
        }
    } else if (early_v) {
        wait_vmcnt<0>();
        __syncthreads();                  // the key rows (and the roped q and k) are in
        if (is_k && pos >= 0 && pos < vis) {
#pragma unroll
            for (int u = 0; u < kPer; ++u) {
                const int i = lane + 64 * u;
                vs[(size_t)pos * D + 8 * ((i / 8) ^ (pos & (per_row - 1))) + i % 8] = kb[u];
            }
        }
        __syncthreads();
        uint32_t ka[D / 2];
        if (t < vis) {
            const uint16_t *row = vs + (size_t)t * D;
#pragma unroll
            for (int u = 0; u < per_row; ++u) {
                const u32x4 c = *(const u32x4 *)(row + 8 * (u ^ (t & (per_row - 1))));
                ka[4 * u] = c[0];
                ka[4 * u + 1] = c[1];
                ka[4 * u + 2] = c[2];
                ka[4 * u + 3] = c[3];
            }
        }
        __syncthreads();                  // every key row is out of the staging
        stage(v_cache, 0, false);         // value rows arrive during the scores and the softmax
        if (t < vis) {
#pragma unroll
            for (int r = 0; r < hpw; ++r)
                sc[(size_t)r * scs + t] = bfr(bfr(score_dot<D>(qs + r * D, ka, naive)) * scale);
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   // every score is in
    } else {
        for (int j0 = 0; j0 < vis; j0 += vcap) {
            if (j0 > 0) {
                __syncthreads();              // the previous rows have been read
                stage(k_cache, j0, true);
            }
            wait_vmcnt<0>();
            __syncthreads();                  // the key rows (and the roped q and k) are in
            const int j1 = min(vis, j0 + vcap);
            if (is_k && pos >= j0 && pos < j1) {
                const int jr = pos - j0;
#pragma unroll
                for (int u = 0; u < kPer; ++u) {
                    const int i = lane + 64 * u;
                    vs[(size_t)jr * D + 8 * ((i / 8) ^ (jr & (per_row - 1))) + i % 8] = kb[u];
                }
            }
            __syncthreads();
            for (int j = j0 + t; j < j1; j += nthreads) {
                uint32_t ka[D / 2];
                const int jr = j - j0;
                const uint16_t *row = vs + (size_t)jr * D;
#pragma unroll
                for (int u = 0; u < per_row; ++u) {
                    const u32x4 c = *(const u32x4 *)(row + 8 * (u ^ (jr & (per_row - 1))));
                    ka[4 * u] = c[0];
                    ka[4 * u + 1] = c[1];
                    ka[4 * u + 2] = c[2];
                    ka[4 * u + 3] = c[3];
                }
#pragma unroll
                for (int r = 0; r < hpw; ++r)
                    sc[(size_t)r * scs + j] = bfr(bfr(score_dot<D>(qs + r * D, ka, naive)) * scale);
            }
        }
        __syncthreads();                      // every score is in; the staged key rows are free
        stage(v_cache, 0, false);             // value rows arrive during the softmax
    }

    // softmax per head: wave r (the split path has its weights)
    for (int r = wave; r < (split_v ? 0 : hpw); r += nthreads / 64) {
        float *x = sc + (size_t)r * scs;
        float mx = -__builtin_inff();
        for (int j = lane; j < vis; j += 64) mx = fmaxf(mx, x[j]);
        mx = wave_max_dpp(mx);
        for (int j = lane; j < vis; j += 64) x[j] = sleef_expf(x[j] - mx);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const float inv = __fdiv_rn(1.0f, exp_sum(x, vis, cache_len, lane));
        for (int j = lane; j < vis; j += 64) x[j] = bfr(x[j] * inv);
    }


    // P.V: thread (chain k, column c), every head of this kv head at once;
    // eight positions of a chain (their value and rep weights) loaded ahead
    const int main_len = naive ? 0 : (cache_len / 4) * 4;
    constexpr int nthr = 4 * D;
    if (split_v) {
        // one pass, one head: thread (chain k, column pair cp), k = t / (D / 2),
        // a wave reading whole value rows as 32-bit pairs; chain k's weights
        // four at a time from cm[k c4 + i] (position k + 4 i)
        wait_vmcnt<0>();
        __syncthreads();                  // the value rows and the weights are in
        if (is_k && pos >= 0 && pos < vis) {
#pragma unroll
            for (int u = 0; u < kPer; ++u) vs[(size_t)pos * D + lane + 64 * u] = vr[u];
        }
        __syncthreads();                  // the new value row replaces the staged copy
        if (t < 2 * D) {
            const int k = t / (D / 2), cp = t % (D / 2);
            const uint32_t *vw = (const uint32_t *)vs + cp;       // vw[j * D / 2]: the pair at position j
            float a0 = 0.0f, a1 = 0.0f;
            auto fma_pos = [&](float w, int j) {
                const uint32_t v = vw[(size_t)j * (D / 2)];
                a0 = __builtin_fmaf(w, bf16_lo(v), a0);
                a1 = __builtin_fmaf(w, bf16_hi(v), a1);
            };
            if (naive) {
                if (k == 0)
                    for (int j = 0; j < vis; ++j) fma_pos(sc[j], j);
            } else {
                const float *wk = cm + k * kC4;
                const int im = max(0, (min(vis, main_len) - k + 3) / 4);   // positions k + 4 i
                int i = 0;
                for (; i + 8 <= im; i += 8) {
                    const float4 wa = *(const float4 *)(wk + i), wb = *(const float4 *)(wk + i + 4);
                    uint32_t v[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) v[u] = vw[(size_t)(k + 4 * (i + u)) * (D / 2)];
                    const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        a0 = __builtin_fmaf(wv[u], bf16_lo(v[u]), a0);
                        a1 = __builtin_fmaf(wv[u], bf16_hi(v[u]), a1);
                    }
                }
                for (; i < im; ++i) fma_pos(wk[i], k + 4 * i);
                if (k == 0)
                    for (int j = main_len; j < vis; ++j) fma_pos(sc[j], j);
            }
            part[k * D + 2 * cp] = a0;
            part[k * D + 2 * cp + 1] = a1;
        }
    }
    for (int base = 0; base < (split_v ? 0 : nthr); base += nthreads) {
        const int i = base + t;
        const bool active = i < nthr;
        const int k = (i / D) & 3, c = i % D;
        float acc[hpw];
#pragma unroll
        for (int r = 0; r < hpw; ++r) acc[r] = 0.0f;
        for (int j0 = 0; j0 < vis; j0 += vcap) {
            if (j0 > 0) {
                __syncthreads();          // the previous rows have been read
                stage(v_cache, j0, false);
            }
            if (j0 > 0 || base == 0 || vis > vcap) {
                wait_vmcnt<0>();
                __syncthreads();          // every wave's copies (and the weights) are in
                if (is_k && pos >= j0 && pos < min(vis, j0 + vcap)) {
#pragma unroll
                    for (int u = 0; u < kPer; ++u) vs[(size_t)(pos - j0) * D + lane + 64 * u] = vr[u];
                }
                __syncthreads();          // the new value row replaces the staged copy
            }
            const int j1 = min(vis, j0 + vcap);
            if (active) {
                const uint16_t *vc = vs + c - (size_t)j0 * D;     // vc[j * D]: column c of position j
                auto fma_row = [&](int j) {
                    const float vv = bf(vc[(size_t)j * D]);
#pragma unroll
                    for (int r = 0; r < hpw; ++r) acc[r] = __builtin_fmaf(sc[(size_t)r * scs + j], vv, acc[r]);
                };
                if (naive) {
                    if (k == 0)
                        for (int j = j0; j < j1; ++j) fma_row(j);
                } else {
                    int j = j0 + ((k - j0) & 3);
                    const int jm = min(j1, main_len);
                    for (; j + 28 < jm; j += 32) {
                        float vv[8], wv[8][hpw];
#pragma unroll
                        for (int u = 0; u < 8; ++u) {
                            vv[u] = bf(vc[(size_t)(j + 4 * u) * D]);
#pragma unroll
                            for (int r = 0; r < hpw; ++r) wv[u][r] = sc[(size_t)r * scs + j + 4 * u];
                        }
#pragma unroll
                        for (int u = 0; u < 8; ++u)
#pragma unroll
                            for (int r = 0; r < hpw; ++r) acc[r] = __builtin_fmaf(wv[u][r], vv[u], acc[r]);
                    }
                    for (; j < jm; j += 4) fma_row(j);
                    if (k == 0)
                        for (j = max(j0, main_len); j < j1; ++j) fma_row(j);
                }
            }
            if (vis > vcap && j0 + vcap >= vis && base + nthreads < nthr) {
                __syncthreads();          // the next pass stages from row 0 again
                stage(v_cache, 0, false);
            }
        }
        if (active)
            for (int r = 0; r < hpw; ++r) part[(size_t)r * 4 * D + i] = acc[r];
    }
    __syncthreads();
    // fold: output (head r, column c) for r * D + c = t + nthreads * it
    for (int o = t, it = 0; o < hpw * D; o += nthreads, ++it) {
        const int r = o / D, c = o % D;
        const float *pp = part + (size_t)r * 4 * D + c;
        float v = naive ? pp[0] : ((pp[0] + pp[D]) + pp[2 * D]) + pp[3 * D];
        v = bfr(v);
        const float g = it == 0 ? gpre[0] : it == 1 ? gpre[1] : bf(qg[(size_t)(h0 + r) * 2 * D + D + c]);
        v = v * bfr(__fdiv_rn(1.0f, 1.0f + sleef_expf(-g)));
        out[(size_t)(h0 + r) * D + c] = f32_to_bf16(v);
    }
}

// ---- SiLU(gate) * up --------------------------------------------------------
// out = bf16(bf16(g / (1 + exp(-g))) * u): F.silu(gate) * up on bf16 tensors.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t *__restrict__ g, const uint16_t *__restrict__ u,
                                                       size_t in_stride, uint16_t *__restrict__ out, int n,
                                                       int rows) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)n * rows) return;
    const size_t m = i / n, c = i % n;
    const float gv = bf(g[m * in_stride + c]);
    const float sl = bfr(__fdiv_rn(gv, 1.0f + sleef_expf(-gv)));
    out[i] = f32_to_bf16(sl * bf(u[m * in_stride + c]));
}

// ---- greedy step ------------------------------------------------------------
// argmax of bf16 logits as the first index of the largest value (torch.argmax
// on the fp32 copy, for finite logits): every position becomes the 64-bit key
// (order-preserving bits of the value) << 32 | (2^32 - 1 - index), whose
// maximum is that position; workgroups fold 16-byte loads of logits into a
// key and atomically raise one shared key.  The advance kernel reads it,
// clears it for the next call and moves the decode state on:
// tokens[count] = id, next_id = id, pos0 = cache_len, cache_len += 1,
// count += 1.
__device__ __forceinline__ unsigned long long arg_key(float v, uint32_t idx) {
    const uint32_t b = __float_as_uint(v);
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)o << 32) | (0xFFFFFFFFu - idx);
}

__device__ __forceinline__ unsigned long long max_u64(unsigned long long a, unsigned long long b) {
    return a > b ? a : b;
}

__global__ __launch_bounds__(256) void argmax_key_kernel(const uint16_t *__restrict__ logits, int n,
                                                         unsigned long long *__restrict__ key) {
    const int chunks = n / 8;
    unsigned long long best = 0;
    for (int c = blockIdx.x * 256 + threadIdx.x; c < chunks; c += gridDim.x * 256) {
        const u32x4 v = ((const u32x4 *)logits)[c];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            best = max_u64(best, arg_key(bf16_lo(v[e]), (uint32_t)(8 * c + 2 * e)));
            best = max_u64(best, arg_key(bf16_hi(v[e]), (uint32_t)(8 * c + 2 * e + 1)));
        }
    }
    if (blockIdx.x == 0)
        for (int i = chunks * 8 + threadIdx.x; i < n; i += 256) best = max_u64(best, arg_key(bf(logits[i]), (uint32_t)i));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = ((unsigned long long)(uint32_t)__shfl_xor((int)(best >> 32), off) << 32) |
                                     (uint32_t)__shfl_xor((int)(uint32_t)best, off);
        best = max_u64(best, o);
    }
    // one atomic per workgroup (the key's maximum does not depend on the order)
    __shared__ unsigned long long wbest[4];
    if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_fetch_max(key, max_u64(max_u64(wbest[0], wbest[1]), max_u64(wbest[2], wbest[3])),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ __launch_bounds__(64) void greedy_advance_kernel(unsigned long long *__restrict__ key,
                                                            int32_t *__restrict__ state, int32_t *__restrict__ tokens,
                                                            int64_t *__restrict__ next_id, int max_tokens) {
    if (threadIdx.x != 0) return;
    const unsigned long long k = __hip_atomic_load(key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int id = k ? (int)(0xFFFFFFFFu - (uint32_t)k) : 0;
    __hip_atomic_store(key, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int count = state[2];
    if (count < max_tokens) tokens[count] = id;
    state[2] = count + 1;
    next_id[0] = id;
    state[0] = state[1];
    state[1] = state[1] + 1;
}

// The batch rows of a table of sequences: every row of [0, total) belongs
// to exactly one sequence, whose positions fit max_len and whose table
// index is below n_tables.
int build_batch_rows(const ekernel_batch_seq_t *seqs, size_t n_seqs, size_t total, size_t n_tables,
                     size_t n_block_ids, size_t max_len, BatchRows &br, const char *fn) {
    if (!seqs || n_seqs == 0) return fail(ECPU_ERR_PARAM, "%s: no sequences", fn);
    if (total > (size_t)kMaxBatchRows)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: %zu rows in one call (at most %d)", fn, total, kMaxBatchRows);
    for (int r = 0; r < kMaxBatchRows; ++r) br.nrows[r] = 0;
    for (size_t i = 0; i < n_seqs; ++i) {
        const ekernel_batch_seq_t &q = seqs[i];
        if (q.row0 < 0 || q.rows < 1 || (size_t)q.row0 + (size_t)q.rows > total)
            return fail(ECPU_ERR_PARAM, "%s: sequence %zu: rows %d..%d outside the %zu batch rows", fn, i, q.row0,
                        q.row0 + q.rows - 1, total);
        if (q.pos0 < 0 || (size_t)q.pos0 + (size_t)q.rows > max_len)
            return fail(ECPU_ERR_PARAM, "%s: sequence %zu: positions %d..%d beyond the %zu its tables hold", fn, i,
                        q.pos0, q.pos0 + q.rows - 1, max_len);
        if (q.table < 0 || (size_t)q.table >= n_tables)
            return fail(ECPU_ERR_PARAM, "%s: sequence %zu: table %d of %zu", fn, i, q.table, n_tables);
        for (int u = 0; u < q.rows; ++u) {
            const int r = q.row0 + u;
            if (br.nrows[r] != 0) return fail(ECPU_ERR_PARAM, "%s: batch row %d in two sequences", fn, r);
            br.pos[r] = q.pos0 + u;
            br.len[r] = q.pos0 + q.rows;
            br.nrows[r] = q.rows;
            br.tbl[r] = (int32_t)((size_t)q.table * n_block_ids);
        }
    }
    for (size_t r = 0; r < total; ++r)
        if (br.nrows[r] == 0) return fail(ECPU_ERR_PARAM, "%s: batch row %zu belongs to no sequence", fn, r);
    return ECPU_OK;
}

}  // namespace

}  // namespace pilm

using namespace pilm;

extern "C" {

int ekernel_rmsnorm_gemma_bf16(const ekernel_rmsnorm_desc_t *desc, const uint16_t *x, const uint16_t *residual,
                               const uint16_t *weight, uint16_t *out, uint16_t *residual_out) {
    static const char *fn = "ekernel_rmsnorm_gemma_bf16";
    if (!desc || !x || !weight || !out) return fail(ECPU_ERR_PARAM, "%s: null argument", fn);
    const size_t M = desc->rows, n = desc->hidden;
    if (M == 0) return ECPU_OK;
    if (n < 32 || n > 8192) return fail(ECPU_ERR_UNSUPPORTED, "%s: hidden %zu outside [32, 8192]", fn, n);
    const size_t bytes = M * n * 2;
    int rc = check_device_buffer(x, bytes, "x", fn);
    if (rc == ECPU_OK && residual) rc = check_device_buffer(residual, bytes, "residual", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(weight, n * 2, "weight", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(out, bytes, "out", fn);
    if (rc == ECPU_OK && residual_out) rc = check_device_buffer(residual_out, bytes, "residual_out", fn);
    if (rc != ECPU_OK) return rc;
    const size_t lds = (n + 4 + 32 * (n / 512 + 1)) * sizeof(float);   // row, r, block sums
    const uintptr_t ptrs = (uintptr_t)x | (uintptr_t)residual | (uintptr_t)weight | (uintptr_t)out |
                           (uintptr_t)residual_out;
    hipStream_t st = current_stream();
    if (n % 8 == 0 && (ptrs & 15) == 0) {
        if (n <= 2048)
            rmsnorm_vec_kernel<1><<<(unsigned)M, 256, lds, st>>>(x, residual, weight, out, residual_out, (int)n,
                                                                 desc->eps);
        else if (n <= 4096)
            rmsnorm_vec_kernel<2><<<(unsigned)M, 256, lds, st>>>(x, residual, weight, out, residual_out, (int)n,
                                                                 desc->eps);
        else
            rmsnorm_vec_kernel<4><<<(unsigned)M, 256, lds, st>>>(x, residual, weight, out, residual_out, (int)n,
                                                                 desc->eps);
    } else {
        rmsnorm_kernel<<<(unsigned)M, 256, lds, st>>>(x, residual, weight, out, residual_out, (int)n, desc->eps);
    }
    return check_launch(fn);
}

int ekernel_qk_norm_rope_bf16(const ekernel_qk_rope_desc_t *desc, const uint16_t *qg, const uint16_t *k,
                              const uint16_t *v, const uint16_t *q_norm_w, const uint16_t *k_norm_w,
                              const float *cos_table, const float *sin_table, const int32_t *step,
                              uint16_t *q_out, uint16_t *k_cache, uint16_t *v_cache, const int32_t *block_ids) {
    static const char *fn = "ekernel_qk_norm_rope_bf16";
    if (!desc || !qg || !k || !v || !q_norm_w || !k_norm_w || !cos_table || !sin_table || !q_out || !k_cache ||
        !v_cache || !block_ids)
        return fail(ECPU_ERR_PARAM, "%s: null argument", fn);
    const ekernel_qk_rope_desc_t &d = *desc;
    if (d.S == 0) return ECPU_OK;
    if (d.head_dim < 32 || d.head_dim > 256 || d.head_dim % 8 || d.rot_dim > d.head_dim || d.rot_dim % 2 ||
        d.n_kv_heads == 0 || d.n_heads % d.n_kv_heads || d.block_size == 0 || d.n_block_ids == 0 ||
        d.max_positions == 0)
        return fail(ECPU_ERR_PARAM, "%s: inconsistent descriptor", fn);
    if (!step && (d.pos0 + d.S > d.max_positions || d.pos0 + d.S > d.n_block_ids * d.block_size))
        return fail(ECPU_ERR_PARAM, "%s: positions %zu..%zu beyond the tables", fn, d.pos0, d.pos0 + d.S - 1);
    const size_t D = d.head_dim;
    int rc = check_device_buffer(q_out, d.S * d.n_heads * D * 2, "q_out", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(k_cache, d.num_blocks * d.block_size * d.n_kv_heads * D * 2, "k_cache", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(v_cache, d.num_blocks * d.block_size * d.n_kv_heads * D * 2, "v_cache", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(block_ids, d.n_block_ids * 4, "block_ids", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(cos_table, d.max_positions * (d.rot_dim / 2) * 4, "cos_table", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(sin_table, d.max_positions * (d.rot_dim / 2) * 4, "sin_table", fn);
    if (rc != ECPU_OK) return rc;
    const dim3 grid((unsigned)d.S, (unsigned)(d.n_heads + d.n_kv_heads));
    qk_rope_kernel<OneSeq><<<grid, 64, 0, current_stream()>>>(
        qg, k, v, d.q_stride, d.kv_stride, q_norm_w, k_norm_w, cos_table, sin_table, (int)d.max_positions, step, (int)d.pos0,
        q_out, k_cache, v_cache, block_ids, (int)d.n_block_ids, (int)d.block_size, (int)d.num_blocks,
        (int)d.n_heads, (int)d.n_kv_heads, (int)D, (int)d.rot_dim, d.eps, OneSeq{});
    return check_launch(fn);
}

int ekernel_attention_exact_bf16(const ekernel_attention_exact_desc_t *desc, const uint16_t *q,
                                 const uint16_t *k_cache, const uint16_t *v_cache, const int32_t *block_ids,
                                 const uint16_t *gate, const int32_t *step, uint16_t *out) {
    static const char *fn = "ekernel_attention_exact_bf16";
    if (!desc || !q || !k_cache || !v_cache || !block_ids || !out)
        return fail(ECPU_ERR_PARAM, "%s: null argument", fn);
    const ekernel_attention_exact_desc_t &d = *desc;
    if (d.S == 0) return ECPU_OK;
    if (d.n_kv_heads == 0 || d.n_heads % d.n_kv_heads || d.block_size == 0 || d.n_block_ids == 0)
        return fail(ECPU_ERR_PARAM, "%s: inconsistent descriptor", fn);
    if (d.head_dim != 64 && d.head_dim != 128 && d.head_dim != 256)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: head_dim %zu (64, 128 or 256)", fn, d.head_dim);
    const size_t max_len = d.n_block_ids * d.block_size;
    if (!step && (d.cache_len < d.S || d.cache_len > max_len))
        return fail(ECPU_ERR_PARAM, "%s: cache_len %zu outside [S, %zu]", fn, d.cache_len, max_len);
    const size_t rep = d.n_heads / d.n_kv_heads, D = d.head_dim;
    const size_t fixed = (rep * D + rep * ((max_len + 3) & ~(size_t)3) + rep * kDS * 4 +
                          ((d.n_block_ids + 3) & ~(size_t)3)) * 4;
    // value rows staged per pass: all of them when they fit, in 64-row steps
    const size_t room = fixed < 64 * 1024 ? (64 * 1024 - fixed) / (kDS * 2) : 0;
    const size_t vcap = std::min<size_t>(room / 64 * 64, (max_len + 63) / 64 * 64);
    if (vcap < 64)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: %zu positions x %zu heads per kv head exceed LDS", fn, max_len, rep);
    const size_t lds = fixed + vcap * kDS * 2;
    const size_t cache_bytes = d.num_blocks * d.block_size * d.n_kv_heads * D * 2;
    int rc = check_device_buffer(q, d.S * d.n_heads * D * 2, "q", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(k_cache, cache_bytes, "k_cache", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(v_cache, cache_bytes, "v_cache", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(block_ids, d.n_block_ids * 4, "block_ids", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(out, d.S * d.n_heads * D * 2, "out", fn);
    if (rc != ECPU_OK) return rc;
    const dim3 grid((unsigned)d.n_kv_heads, (unsigned)d.S, (unsigned)(D / kDS));
    const float scale = (float)(1.0 / __builtin_sqrt((double)D));
    hipStream_t st = current_stream();
#define PILM_ATTN_EXACT(DD)                                                                                         \
    attn_exact_kernel<DD, OneSeq><<<grid, 256, lds, st>>>(q, k_cache, v_cache, block_ids, (int)d.n_block_ids,     \
                                                          (int)d.num_blocks, (int)d.block_size, gate,               \
                                                          d.gate_row_stride, d.gate_head_stride, step,              \
                                                          (int)d.cache_len, (int)d.S, (int)d.n_heads,               \
                                                          (int)d.n_kv_heads, (int)max_len, (int)vcap, scale, out,   \
                                                          OneSeq{})
    if (D == 64) PILM_ATTN_EXACT(64);
    else if (D == 128) PILM_ATTN_EXACT(128);
    else PILM_ATTN_EXACT(256);
#undef PILM_ATTN_EXACT
    return check_launch(fn);
}

int ekernel_qk_norm_rope_batch_bf16(const ekernel_qk_rope_desc_t *desc, const ekernel_batch_seq_t *seqs,
                                    size_t n_seqs, size_t n_tables, const uint16_t *qg, const uint16_t *k,
                                    const uint16_t *v, const uint16_t *q_norm_w, const uint16_t *k_norm_w,
                                    const float *cos_table, const float *sin_table, uint16_t *q_out,
                                    uint16_t *k_cache, uint16_t *v_cache, const int32_t *block_ids) {
    static const char *fn = "ekernel_qk_norm_rope_batch_bf16";
    if (!desc || !qg || !k || !v || !q_norm_w || !k_norm_w || !cos_table || !sin_table || !q_out || !k_cache ||
        !v_cache || !block_ids)
        return fail(ECPU_ERR_PARAM, "%s: null argument", fn);
    const ekernel_qk_rope_desc_t &d = *desc;
    if (d.S == 0) return ECPU_OK;
    if (d.head_dim < 32 || d.head_dim > 256 || d.head_dim % 8 || d.rot_dim > d.head_dim || d.rot_dim % 2 ||
        d.n_kv_heads == 0 || d.n_heads % d.n_kv_heads || d.block_size == 0 || d.n_block_ids == 0 ||
        d.max_positions == 0)
        return fail(ECPU_ERR_PARAM, "%s: inconsistent descriptor", fn);
    BatchRows br;
    const size_t max_len = std::min(d.max_positions, d.n_block_ids * d.block_size);
    int rc = build_batch_rows(seqs, n_seqs, d.S, n_tables, d.n_block_ids, max_len, br, fn);
    if (rc != ECPU_OK) return rc;
    const size_t D = d.head_dim;
    rc = check_device_buffer(q_out, d.S * d.n_heads * D * 2, "q_out", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(k_cache, d.num_blocks * d.block_size * d.n_kv_heads * D * 2, "k_cache", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(v_cache, d.num_blocks * d.block_size * d.n_kv_heads * D * 2, "v_cache", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(block_ids, n_tables * d.n_block_ids * 4, "block_ids", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(cos_table, d.max_positions * (d.rot_dim / 2) * 4, "cos_table", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(sin_table, d.max_positions * (d.rot_dim / 2) * 4, "sin_table", fn);
    if (rc != ECPU_OK) return rc;
    const dim3 grid((unsigned)d.S, (unsigned)(d.n_heads + d.n_kv_heads));
    qk_rope_kernel<BatchRows><<<grid, 64, 0, current_stream()>>>(
        qg, k, v, d.q_stride, d.kv_stride, q_norm_w, k_norm_w, cos_table, sin_table, (int)d.max_positions, nullptr,
        0, q_out, k_cache, v_cache, block_ids, (int)d.n_block_ids, (int)d.block_size, (int)d.num_blocks,
        (int)d.n_heads, (int)d.n_kv_heads, (int)D, (int)d.rot_dim, d.eps, br);
    return check_launch(fn);
}

static size_t lds_limit();

int ekernel_attention_exact_batch_bf16(const ekernel_attention_exact_desc_t *desc, const ekernel_batch_seq_t *seqs,
                                       size_t n_seqs, size_t n_tables, const uint16_t *q, const uint16_t *k_cache,
                                       const uint16_t *v_cache, const int32_t *block_ids, const uint16_t *gate,
                                       uint16_t *out) {
    static const char *fn = "ekernel_attention_exact_batch_bf16";
    if (!desc || !q || !k_cache || !v_cache || !block_ids || !out)
        return fail(ECPU_ERR_PARAM, "%s: null argument", fn);
    const ekernel_attention_exact_desc_t &d = *desc;
    if (d.S == 0) return ECPU_OK;
    if (d.n_kv_heads == 0 || d.n_heads % d.n_kv_heads || d.block_size == 0 || d.n_block_ids == 0)
        return fail(ECPU_ERR_PARAM, "%s: inconsistent descriptor", fn);
    if (d.head_dim != 64 && d.head_dim != 128 && d.head_dim != 256)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: head_dim %zu (64, 128 or 256)", fn, d.head_dim);
    const size_t max_len = d.n_block_ids * d.block_size;
    BatchRows br;
    int rc = build_batch_rows(seqs, n_seqs, d.S, n_tables, d.n_block_ids, max_len, br, fn);
    if (rc != ECPU_OK) return rc;
    const size_t rep = d.n_heads / d.n_kv_heads, D = d.head_dim;
    const size_t cache_bytes = d.num_blocks * d.block_size * d.n_kv_heads * D * 2;
    rc = check_device_buffer(q, d.S * d.n_heads * D * 2, "q", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(k_cache, cache_bytes, "k_cache", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(v_cache, cache_bytes, "v_cache", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(block_ids, n_tables * d.n_block_ids * 4, "block_ids", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(out, d.S * d.n_heads * D * 2, "out", fn);
    if (rc != ECPU_OK) return rc;
    const float scale = (float)(1.0 / __builtin_sqrt((double)D));
    hipStream_t st = current_stream();
    if ((D == 64 || D == 128) && rep <= (size_t)kTileVecs && env_int("PILM_HIP_ATTN_TILE", 1) != 0) {
        // tiles of at most rt rows per sequence: the most rows per tile that
        // still give 256 workgroups (else one row per tile), fewer if the
        // scores do not fit the workgroup's LDS
        int longest = 1, most = 1;
        for (size_t i = 0; i < n_seqs; ++i) {
            longest = std::max(longest, seqs[i].pos0 + seqs[i].rows);
            most = std::max(most, seqs[i].rows);
        }
        const int rt_max = std::min((int)(kTileVecs / rep), most);
        int rt = env_int("PILM_HIP_ATTN_TILE_ROWS", 0);
        if (rt <= 0) {
            rt = 1;
            for (int c = rt_max; c > 1; --c) {
                size_t n = 0;
                for (size_t i = 0; i < n_seqs; ++i) n += (size_t)(seqs[i].rows + c - 1) / c;
                if (n * d.n_kv_heads >= 256) {
                    rt = c;
                    break;
                }
            }
        }
        const size_t scs = ((size_t)longest + 3) & ~(size_t)3, budget = lds_limit();
        for (rt = std::min(rt, rt_max); rt >= 1; --rt) {
            BatchTiles bt;
            int n_tiles = 0, widest = 0;
            for (size_t i = 0; i < n_seqs; ++i) {
                const int nrow = seqs[i].rows, nt = (nrow + rt - 1) / rt, per = (nrow + nt - 1) / nt;
                for (int r = 0; r < nrow; r += per) {
                    const int m = std::min(per, nrow - r);
                    bt.tile[n_tiles++] = (seqs[i].row0 + r) | (m << 16);
                    widest = std::max(widest, m);
                }
            }
            const size_t vecs = (size_t)widest * rep;
            const size_t fixed = (vecs * (D + 4) + vecs * scs + ((d.n_block_ids + 3) & ~(size_t)3)) * 4;
            if (fixed >= budget) continue;
            const size_t vcap = std::min((budget - fixed) / (D * 2) / 64 * 64, ((size_t)longest + 63) / 64 * 64);
            if (vcap < 64) continue;
            const size_t lds = fixed + vcap * D * 2;
            const dim3 tgrid((unsigned)d.n_kv_heads, (unsigned)n_tiles);
            // vectors per P.V thread: the widest tile's over the vector groups
            const int nv = (int)((vecs + (kTileThreads / (2 * D)) - 1) / (kTileThreads / (2 * D)));
#define PILM_ATTN_TILE(DD, NVV)                                                                                     \
    attn_tile_kernel<DD, NVV><<<tgrid, kTileThreads, lds, st>>>(                                                    \
        q, k_cache, v_cache, block_ids, (int)d.n_block_ids, (int)d.num_blocks, (int)d.block_size, gate,             \
        d.gate_row_stride, d.gate_head_stride, (int)d.n_heads, (int)d.n_kv_heads, (int)max_len, (int)vecs,          \
        (int)scs, (int)vcap, scale, out, br, bt)
            if (D == 64) {
                switch (nv) {
                case 1: PILM_ATTN_TILE(64, 1); break;
                case 2: PILM_ATTN_TILE(64, 2); break;
                case 3: PILM_ATTN_TILE(64, 3); break;
                default: PILM_ATTN_TILE(64, 4); break;
                }
            } else {
                switch (nv) {
                case 1: PILM_ATTN_TILE(128, 1); break;
                case 2: PILM_ATTN_TILE(128, 2); break;
                case 3: PILM_ATTN_TILE(128, 3); break;
                case 4: PILM_ATTN_TILE(128, 4); break;
                case 5: PILM_ATTN_TILE(128, 5); break;
                case 6: PILM_ATTN_TILE(128, 6); break;
                case 7: PILM_ATTN_TILE(128, 7); break;
                default: PILM_ATTN_TILE(128, 8); break;
                }
            }
#undef PILM_ATTN_TILE
            return check_launch(fn);
        }
    }
    // the per-row kernel: value rows staged per pass, all of them when they fit
    const size_t fixed = (rep * D + rep * ((max_len + 3) & ~(size_t)3) + rep * kDS * 4 +
                          ((d.n_block_ids + 3) & ~(size_t)3)) * 4;
    const size_t room = fixed < 64 * 1024 ? (64 * 1024 - fixed) / (kDS * 2) : 0;
    const size_t vcap = std::min<size_t>(room / 64 * 64, (max_len + 63) / 64 * 64);
    if (vcap < 64)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: %zu positions x %zu heads per kv head exceed LDS", fn, max_len, rep);
    const size_t lds = fixed + vcap * kDS * 2;
    const dim3 grid((unsigned)d.n_kv_heads, (unsigned)d.S, (unsigned)(D / kDS));
#define PILM_ATTN_BATCH(DD)                                                                                       \
    attn_exact_kernel<DD, BatchRows><<<grid, 256, lds, st>>>(q, k_cache, v_cache, block_ids, (int)d.n_block_ids,  \
                                                             (int)d.num_blocks, (int)d.block_size, gate,            \
                                                             d.gate_row_stride, d.gate_head_stride, nullptr, 0, 0,  \
                                                             (int)d.n_heads, (int)d.n_kv_heads, (int)max_len,       \
                                                             (int)vcap, scale, out, br)
    if (D == 64) PILM_ATTN_BATCH(64);
    else if (D == 128) PILM_ATTN_BATCH(128);
    else PILM_ATTN_BATCH(256);
#undef PILM_ATTN_BATCH
    return check_launch(fn);
}

// LDS a workgroup may hold on the current device (gfx950: 160 KB).
static size_t lds_limit() {
    static size_t cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 64 * 1024;
    if (!cached[dev]) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            v = 64 * 1024;
        cached[dev] = std::min<size_t>((size_t)v, 160 * 1024);
    }
    return cached[dev];
}

int ekernel_decode_attention_bf16(const ekernel_qk_rope_desc_t *desc, const uint16_t *qg, const uint16_t *k,
                                  const uint16_t *v, const uint16_t *q_norm_w, const uint16_t *k_norm_w,
                                  const float *cos_table, const float *sin_table, const int32_t *step,
                                  uint16_t *k_cache, uint16_t *v_cache, const int32_t *block_ids, uint16_t *out) {
    static const char *fn = "ekernel_decode_attention_bf16";
    if (!desc || !qg || !k || !v || !q_norm_w || !k_norm_w || !cos_table || !sin_table || !k_cache || !v_cache ||
        !block_ids || !out)
        return fail(ECPU_ERR_PARAM, "%s: null argument", fn);
    const ekernel_qk_rope_desc_t &d = *desc;
    if (d.S != 1) return fail(ECPU_ERR_UNSUPPORTED, "%s: one decode row per call (S = %zu)", fn, d.S);
    // 256-wide heads would hold a whole key row and its products beyond the
    // registers a 512-thread workgroup has: the two-call path serves them
    if (d.head_dim != 64 && d.head_dim != 128)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: head_dim %zu (64 or 128)", fn, d.head_dim);
    if (d.rot_dim > d.head_dim || d.rot_dim % 2 || d.n_kv_heads == 0 || d.n_heads % d.n_kv_heads ||
        d.block_size == 0 || d.n_block_ids == 0 || d.max_positions == 0)
        return fail(ECPU_ERR_PARAM, "%s: inconsistent descriptor", fn);
    const size_t rep = d.n_heads / d.n_kv_heads, D = d.head_dim;
    if (rep != 1 && rep != 2 && rep != 4)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: %zu q heads per kv head (1, 2 or 4)", fn, rep);
    const size_t max_len = d.n_block_ids * d.block_size;
    if (!step && (d.pos0 + 1 > d.max_positions || d.pos0 + 1 > max_len))
        return fail(ECPU_ERR_PARAM, "%s: position %zu beyond the tables", fn, d.pos0);
    // heads per workgroup: one (rep workgroups per kv head, each scoring its
    // own q head with q held in registers; measured faster: Qwen3-1.7B decode
    // 796 -> 848 tok/s), or all rep q heads of the kv head sharing the key
    // rows' widening (PILM_DECODE_ATTN_SHARED=1)
    const size_t hpw = env_int("PILM_DECODE_ATTN_SHARED", 0) == 1 ? rep : 1;
    const size_t fixed = ((hpw + 1) * D + hpw * D + hpw * ((max_len + 3) & ~(size_t)3) + kDecodeThreads + 32 +
                          hpw * 4 * D + ((d.n_block_ids + 3) & ~(size_t)3)) * 4;
    const size_t budget = lds_limit();
    const size_t room = fixed < budget ? (budget - fixed) / (D * 2) : 0;
    const size_t vcap = std::min<size_t>(room / 64 * 64, (max_len + 63) / 64 * 64);
    if (vcap < 64)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: %zu positions x %zu heads per kv head exceed LDS", fn, max_len, rep);
    const size_t lds = fixed + vcap * D * 2;
    const size_t cache_bytes = d.num_blocks * d.block_size * d.n_kv_heads * D * 2;
    int rc = check_device_buffer(qg, d.n_heads * 2 * D * 2, "qg", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(k_cache, cache_bytes, "k_cache", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(v_cache, cache_bytes, "v_cache", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(block_ids, d.n_block_ids * 4, "block_ids", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(cos_table, d.max_positions * (d.rot_dim / 2) * 4, "cos_table", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(sin_table, d.max_positions * (d.rot_dim / 2) * 4, "sin_table", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(out, d.n_heads * D * 2, "out", fn);
    if (rc != ECPU_OK) return rc;
    const float scale = (float)(1.0 / __builtin_sqrt((double)D));
    hipStream_t st = current_stream();
    const dim3 grid((unsigned)d.n_kv_heads, (unsigned)(rep / hpw));
#define PILM_DECODE_ATTN_H(DD, RR, HH)                                                                               \
    decode_attn_kernel<DD, RR, HH><<<grid, kDecodeThreads, lds, st>>>(                                               \
        qg, k, v, q_norm_w, k_norm_w, cos_table, sin_table, (int)d.max_positions, step, (int)d.pos0, k_cache,       \
        v_cache, block_ids, (int)d.n_block_ids, (int)d.block_size, (int)d.num_blocks, (int)d.n_heads,              \
        (int)d.n_kv_heads, (int)d.rot_dim, d.eps, (int)max_len, (int)vcap, scale, out)
#define PILM_DECODE_ATTN(DD, RR)                                                                                     \
    do {                                                                                                             \
        if (hpw == 1) PILM_DECODE_ATTN_H(DD, RR, 1);                                                                 \
        else PILM_DECODE_ATTN_H(DD, RR, RR);                                                                         \
    } while (0)
    if (D == 64) {
        if (rep == 1) PILM_DECODE_ATTN(64, 1);
        else if (rep == 2) PILM_DECODE_ATTN(64, 2);
        else PILM_DECODE_ATTN(64, 4);
    } else {
        if (rep == 1) PILM_DECODE_ATTN(128, 1);
        else if (rep == 2) PILM_DECODE_ATTN(128, 2);
        else PILM_DECODE_ATTN(128, 4);
    }
#undef PILM_DECODE_ATTN
#undef PILM_DECODE_ATTN_H
    return check_launch(fn);
}

int ekernel_silu_mul_bf16(const uint16_t *gate, const uint16_t *up, size_t rows, size_t n, size_t in_stride,
                          uint16_t *out) {
    static const char *fn = "ekernel_silu_mul_bf16";
    if (!gate || !up || !out) return fail(ECPU_ERR_PARAM, "%s: null argument", fn);
    if (rows == 0 || n == 0) return ECPU_OK;
    if (in_stride < n) return fail(ECPU_ERR_PARAM, "%s: row stride %zu < %zu", fn, in_stride, n);
    const size_t in_bytes = ((rows - 1) * in_stride + n) * 2;
    int rc = check_device_buffer(gate, in_bytes, "gate", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(up, in_bytes, "up", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(out, rows * n * 2, "out", fn);
    if (rc != ECPU_OK) return rc;
    const size_t total = rows * n;
    silu_mul_kernel<<<(unsigned)((total + 255) / 256), 256, 0, current_stream()>>>(gate, up, in_stride, out, (int)n,
                                                                                   (int)rows);
    return check_launch(fn);
}

int ekernel_greedy_step_bf16(const uint16_t *logits, size_t n, int32_t *state, int32_t *tokens, size_t max_tokens,
                             int64_t *next_id) {
    static const char *fn = "ekernel_greedy_step_bf16";
    if (!logits || !state || !tokens || !next_id || n == 0) return fail(ECPU_ERR_PARAM, "%s: null argument", fn);
    if (n >= 0x7FFFFFFFu) return fail(ECPU_ERR_PARAM, "%s: %zu logits", fn, n);
    int rc = check_device_buffer(logits, n * 2, "logits", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(state, 3 * 4, "state", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(tokens, max_tokens * 4, "tokens", fn);
    if (rc == ECPU_OK) rc = check_device_buffer(next_id, 8, "next_id", fn);
    if (rc != ECPU_OK) return rc;
    if (((uintptr_t)logits & 15) != 0) return fail(ECPU_ERR_PARAM, "%s: logits not 16-byte aligned", fn);
    hipStream_t st = current_stream();
    // the shared key: tickets 4092-4093 of the per-device split-K set (zero
    // between calls; the K-split kernels use tickets below 4092)
    float *P = nullptr;
    int *T = nullptr;
    rc = split_scratch(st, 0, 4096, &P, &T, fn);
    if (rc != ECPU_OK) return rc;
    unsigned long long *key = (unsigned long long *)(T + 4092);
    // up to 64 workgroups, each thread a few 16-byte chunks (151936 logits:
    // two per thread)
    const unsigned blocks = (unsigned)std::min<size_t>(64, std::max<size_t>(1, (n / 8 + 255) / 256));
    argmax_key_kernel<<<blocks, 256, 0, st>>>(logits, (int)n, key);
    greedy_advance_kernel<<<1, 64, 0, st>>>(key, state, tokens, next_id, (int)max_tokens);
    return check_launch(fn);
}

}  // extern "C"
