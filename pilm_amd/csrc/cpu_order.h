// Device restatements of the torch CPU roundings the decoder keeps (piLM runs
// these steps in torch on the CPU): bf16 widening and rounding, a correctly
// rounded square root, SLEEF's expf_u10, torch's row sum of squares order and
// GemmaRMSNorm's output rounding.  Shared by the decoder kernels and the GEMV
// kernels that take a GemmaRMSNorm prologue.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "gemv_device.h"

#pragma clang fp contract(off)

namespace pilm {

__device__ __forceinline__ float bf(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ float bfr(float x) { return bf(f32_to_bf16(x)); }   // round to bf16, as float
__device__ __forceinline__ float sq(float x) { return x * x; }

// Correctly rounded square root of a positive normal float.  v_sqrt_f32 is
// within one ulp of it; of s and its two neighbours, the residuals
// x - s_dn * s and x - s_up * s (exact through FMA) decide which one the true
// root rounds to, as in the correctly rounded sqrt expansions.
__device__ __forceinline__ float sqrt_rn(float x) {
    const float s = __builtin_amdgcn_sqrtf(x);
    const float dn = __int_as_float(__float_as_int(s) - 1);
    const float up = __int_as_float(__float_as_int(s) + 1);
    float r = s;
    if (__builtin_fmaf(-dn, s, x) <= 0.0f) r = dn;
    if (__builtin_fmaf(-up, s, x) > 0.0f) r = up;
    return r;
}

// SLEEF expf_u10 (sleefsimdsp.c xexpf): q = rint(d / ln 2), Cody-Waite
// reduction with the two-part ln 2, a degree-6 polynomial in FMA Horner form,
// 1 + s + s^2 u, scaled by 2^q in two halves; 0 below -104, inf above 100.
__device__ __forceinline__ float sleef_expf(float d) {
    const float q = rintf(d * 1.442695040888963407359924681001892137426645954152985934135449406931f);
    const int qi = (int)q;
    float s = __builtin_fmaf(q, -0.693145751953125f, d);
    s = __builtin_fmaf(q, -1.428606765330187045e-06f, s);
    float u = 0.000198527617612853646278381f;
    u = __builtin_fmaf(u, s, 0.00139304355252534151077271f);
    u = __builtin_fmaf(u, s, 0.00833336077630519866943359f);
    u = __builtin_fmaf(u, s, 0.0416664853692054748535156f);
    u = __builtin_fmaf(u, s, 0.166666671633720397949219f);
    u = __builtin_fmaf(u, s, 0.5f);
    const float ss = s * s;
    u = 1.0f + __builtin_fmaf(ss, u, s);
    const int q1 = qi >> 1;
    u = u * __int_as_float((q1 + 127) << 23);
    u = u * __int_as_float((qi - q1 + 127) << 23);
    if (d < -104.0f) u = 0.0f;
    if (d > 100.0f) u = __builtin_inff();
    return u;
}

// One chain of torch's row sum of squares (x.pow(2).sum(-1) over n >= 32
// contiguous fp32 values in LDS; the squares of bf16 values are exact, as
// x.pow(2) stores them).  Chain t (t < 32) owns lane l = t & 7 of the
// eight-float vectors v = 4r + k, k = t >> 3, accumulated through the cascade
// of 16-row levels; the vectors the four-way interleave leaves over go to
// chain group k = 0.  Loads are issued 16 at a time ahead of their sums.
__device__ inline float chain_sumsq(const float *x, int n, int t) {
    const int k = t >> 3, l = t & 7;
    const int nvec = n / 8, size_ilp = nvec / 4;
    int clog = 0;
    while ((1 << clog) < size_ilp) ++clog;
    const int level_power = max(4, clog / 4);
    const int step = 1 << level_power, mask = step - 1;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int r = 0;
    while (r + step <= size_ilp) {
        for (int j0 = 0; j0 < step; j0 += 16) {
            float v[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = x[8 * (4 * (r + j) + k) + l];
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[0] = acc[0] + sq(v[j]);
            r += 16;
        }
        for (int j = 1; j < 4; ++j) {
            acc[j] = acc[j] + acc[j - 1];
            acc[j - 1] = 0.0f;
            if ((r & (mask << (j * level_power))) != 0) break;
        }
    }
    for (; r < size_ilp; ++r) acc[0] = acc[0] + sq(x[8 * (4 * r + k) + l]);
    float a = acc[0];
    for (int j = 1; j < 4; ++j) a = a + acc[j];
    if (k == 0)
        for (int v = 4 * size_ilp; v < nvec; ++v) a = a + sq(x[8 * v + l]);
    return a;
}

// The chains' lanes folded ((c0 + c1) + c2) + c3 across the four chain
// groups, then the scalar tail and the eight lanes added to 0 in order --
// torch's sum -- divided by n: 1 / sqrt(mean + eps).  c: chain `lane` on
// lanes 0..31 of a whole wave (every lane gets the result).
__device__ inline float fold_row_rsqrt(float c, const float *x, int n, float eps) {
    const int l = (threadIdx.x & 63) & 7;
    const float p = ((c + __shfl(c, l + 8)) + __shfl(c, l + 16)) + __shfl(c, l + 24);
    float fin = 0.0f;
    for (int i = (n / 8) * 8; i < n; ++i) fin = fin + sq(x[i]);
#pragma unroll
    for (int j = 0; j < 8; ++j) fin = fin + __shfl(p, j);
    return __fdiv_rn(1.0f, sqrt_rn(__fdiv_rn(fin, (float)n) + eps));
}

// 1 / sqrt(mean(x^2) + eps) of a row in LDS, computed by one whole wave
// (every lane gets it): the 32 chains, then fold_row_rsqrt.
__device__ inline float wave_row_rsqrt(const float *x, int n, float eps) {
    const int lane = threadIdx.x & 63;
    const float c = lane < 32 ? chain_sumsq(x, n, lane) : 0.0f;
    return fold_row_rsqrt(c, x, n, eps);
}

// The same result with the work spread over a workgroup, for rows with
// n % 32 == 0 and n <= 16384 (then every chain is a run of 16-vector blocks,
// each summed from 0, and the cascade's level step is 16 blocks' worth of
// vectors: level_power 4 in chain_sumsq).  Part one, every thread of the
// workgroup: block sum b of chain t into bs[32 b + t] (b < nblk), and the
// chain's remainder (its last size_ilp % 16 vectors, summed from 0) into
// bs[32 nblk + t].  bs holds 32 (n / 512 + 1) floats.
__device__ inline void row_sumsq_blocks(const float *x, int n, float *bs, int tid, int nthr) {
    const int size_ilp = n / 32, nblk = size_ilp / 16, rem = size_ilp - 16 * nblk;
    const int nb = 32 * (nblk + (rem ? 1 : 0));
    for (int i = tid; i < nb; i += nthr) {
        const int t = i & 31, b = i >> 5, k = t >> 3, l = t & 7;
        const int len = b < nblk ? 16 : rem;
        float a = 0.0f;
        for (int j = 0; j < len; ++j) a = a + sq(x[8 * (4 * (16 * b + j) + k) + l]);
        bs[i] = a;
    }
}

// Part two, one whole wave after the block sums are in: each chain replays
// chain_sumsq's cascade over its block sums (acc[1] += block; at every 256
// vectors acc[2] += acc[1], at every 4096 acc[3] += acc[2]), adds its
// remainder as acc[0], then fold_row_rsqrt.
__device__ inline float wave_row_rsqrt_blocks(const float *x, const float *bs, int n, float eps) {
    const int lane = threadIdx.x & 63;
    const int size_ilp = n / 32, nblk = size_ilp / 16, rem = size_ilp - 16 * nblk;
    float c = 0.0f;
    if (lane < 32) {
        float a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        for (int b = 0; b < nblk; ++b) {
            const int r = 16 * (b + 1);
            a1 = a1 + bs[32 * b + lane];
            if ((r & (15 << 4)) == 0) {
                a2 = a2 + a1;
                a1 = 0.0f;
                if ((r & (15 << 8)) == 0) {
                    a3 = a3 + a2;
                    a2 = 0.0f;
                }
            }
        }
        const float a0 = rem ? bs[32 * nblk + lane] : 0.0f;
        c = ((a0 + a1) + a2) + a3;
    }
    return fold_row_rsqrt(c, x, n, eps);
}

// GemmaRMSNorm (layers.py:130-147) output of one element: bf16((w + 1) *
// bf16(h * r)).
__device__ __forceinline__ uint16_t gemma_out(float h, float r, uint16_t w) {
    return f32_to_bf16(bfr(bf(w) + 1.0f) * bfr(h * r));
}

}  // namespace pilm
