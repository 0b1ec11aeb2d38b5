/*
 * CPU oracle for the quantized matrix-product path -- TEST INFRASTRUCTURE.
 *
 * This file restates, in plain scalar C, the arithmetic of the reference's
 * CPU kernels so that the HIP product can be checked bit for bit.  It is
 * linked only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg, always to compare against and never as the thing measured or shipped.
 *
 * Reference (paths relative to the piLM repository):
 *   src/ecpu/src/kernel/kernels.c
 *     12-25    bf16_to_f32 / f32_to_bf16 (round to nearest even, no NaN case)
 *     43-46    unpack_i4_signed (two's-complement nibble, low nibble = even k)
 *     56-63    hsum256_ps  -> ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7))
 *     78-91    dot_f32_i8_avx2      (8 fp32 FMA lanes, k = l mod 8, scalar tail)
 *     93-109, 278-393  dot_bf16_i8*_avx2 (same lane order, bf16 activations)
 *     111-154, 168-225 dot_bf16_i4*_packed_avx2 (two 8-lane accumulators per
 *              16-element chunk, hsum(lo+hi), scalar tail in pairs)
 *     437-467  ekernel_linear_w8a32
 *     469-656  ekernel_linear_w8a16_bf16
 *     658-737  ekernel_linear_w8a16_bf16_argmax
 *     1002-1087 ekernel_linear_w4a16_bf16
 *     1089-1157 linear_w4a16g_bf16_impl (+ g32 / g128 entry points)
 *     1580-1596 ekernel_swiglu_bf16
 *     1598-1735 ekernel_swiglu_w4a16_bf16
 *
 * The reference is compiled by GCC in GNU C mode with FMA available, where
 * floating-point contraction defaults to "fast": every scalar `s += a * b`
 * in the tails and the group accumulation `acc += block_acc * s[g]` becomes
 * one fused multiply-add.  The restatement spells those as fmaf() and is
 * itself compiled with contraction off.  tests/test_oracle.py pins this
 * against the reference library built from source (oracle/_ref) and against
 * the committed golden vectors.
 */
#include <math.h>
#include <stddef.h>

/* ORACLE_PLANT selects a deliberately wrong variant of the restatement; it is
 * set only by tests/test_oracle.py, which builds each variant into
 * oracle/_build/ and checks that the golden vectors reject it:
 *   1 scalar tails as a*b rounded then added (no FMA)
 *   2 horizontal sum in lane order 0..7
 *   3 group fold as block*scale rounded then added (no FMA)
 *   4 high nibble taken as the even k
 *   5 nibble decoded as v - 8 (a zero point) instead of sign extension
 *   6 bf16 output truncated instead of rounded to nearest even
 *   7 int4 dot with one 8-lane accumulator instead of lo/hi halves
 *   8 SwiGLU gate/up sums scaled but not rounded to bf16 before silu
 *   9 silu(g) with expf(g) instead of expf(-g) */
#ifndef ORACLE_PLANT
#define ORACLE_PLANT 0
#endif
#include <stdint.h>
#include <string.h>

static inline float bf16_to_f32(uint16_t x) {
    uint32_t bits = ((uint32_t)x) << 16;
    float out;
    memcpy(&out, &bits, sizeof(out));
    return out;
}

static inline uint16_t f32_to_bf16(float x) {
    uint32_t bits;
    memcpy(&bits, &x, sizeof(bits));
#if ORACLE_PLANT != 6
    bits += 0x7FFFu + ((bits >> 16) & 1u);
#endif
    return (uint16_t)(bits >> 16);
}

static inline float tail_fma(float a, float b, float acc) {
#if ORACLE_PLANT == 1
    float p = a * b;
    return acc + p;
#else
    return fmaf(a, b, acc);
#endif
}

static inline float nibble_at(const uint8_t *w, size_t k) {
    uint8_t b = w[k >> 1];
#if ORACLE_PLANT == 4
    int v = (k & 1) ? (b & 0x0F) : (b >> 4);
#else
    int v = (k & 1) ? (b >> 4) : (b & 0x0F);
#endif
#if ORACLE_PLANT == 5
    return (float)(v - 8);
#else
    return (float)(v >= 8 ? v - 16 : v);
#endif
}

static inline float hsum8(const float l[8]) {
#if ORACLE_PLANT == 2
    return ((((((l[0] + l[1]) + l[2]) + l[3]) + l[4]) + l[5]) + l[6]) + l[7];
#else
    return ((l[0] + l[4]) + (l[1] + l[5])) + ((l[2] + l[6]) + (l[3] + l[7]));
#endif
}

/* kernels.c:78-91 / 93-109 / 330-393: 8 lanes, lane l owns k = l (mod 8). */
static float dot_i8(const float *a_f32, const uint16_t *a_bf16, const int8_t *w, size_t K) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t k = 0;
    for (; k + 8 <= K; k += 8) {
        for (int l = 0; l < 8; l++) {
            float a = a_f32 ? a_f32[k + l] : bf16_to_f32(a_bf16[k + l]);
            acc[l] = fmaf(a, (float)w[k + l], acc[l]);
        }
    }
    float out = hsum8(acc);
    for (; k < K; k++) {
        float a = a_f32 ? a_f32[k] : bf16_to_f32(a_bf16[k]);
        out = tail_fma(a, (float)w[k], out);
    }
    return out;
}

/* kernels.c:111-154 / 168-225: per 16-chunk, lo lanes take k..k+7 and hi
 * lanes take k+8..k+15; hsum(lo+hi); tail in pairs, then a lone last k. */
static float dot_i4(const uint16_t *a, const uint8_t *w, size_t K) {
    float lo[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float hi[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t k = 0;
    for (; k + 16 <= K; k += 16) {
        for (int l = 0; l < 8; l++) {
            lo[l] = fmaf(bf16_to_f32(a[k + l]), nibble_at(w, k + l), lo[l]);
#if ORACLE_PLANT == 7
            lo[l] = fmaf(bf16_to_f32(a[k + 8 + l]), nibble_at(w, k + 8 + l), lo[l]);
#else
            hi[l] = fmaf(bf16_to_f32(a[k + 8 + l]), nibble_at(w, k + 8 + l), hi[l]);
#endif
        }
    }
    float s[8];
    for (int l = 0; l < 8; l++) s[l] = lo[l] + hi[l];
    float out = hsum8(s);
    for (; k + 1 < K; k += 2) {
        out = tail_fma(bf16_to_f32(a[k]), nibble_at(w, k), out);
        out = tail_fma(bf16_to_f32(a[k + 1]), nibble_at(w, k + 1), out);
    }
    if (k < K) out = tail_fma(bf16_to_f32(a[k]), nibble_at(w, k), out);
    return out;
}

/* kernels.c:437-467 */
int oracle_linear_w8a32(size_t M, size_t N, size_t K, const float *A, const int8_t *W,
                        const float *scales, float *C) {
    if (!A || !W || !scales || !C) return -1;
    #pragma omp parallel for collapse(2) schedule(static)
    for (long long mi = 0; mi < (long long)M; mi++)
        for (long long ni = 0; ni < (long long)N; ni++) {
            float acc = dot_i8(A + (size_t)mi * K, NULL, W + (size_t)ni * K, K);
            C[(size_t)mi * N + (size_t)ni] = acc * scales[ni];
        }
    return 0;
}

/* kernels.c:469-656 (every branch there computes the same per-element value) */
int oracle_linear_w8a16_bf16(size_t M, size_t N, size_t K, const uint16_t *A, const int8_t *W,
                             const float *scales, uint16_t *C) {
    if (!A || !W || !scales || !C) return -1;
    #pragma omp parallel for collapse(2) schedule(static)
    for (long long mi = 0; mi < (long long)M; mi++)
        for (long long ni = 0; ni < (long long)N; ni++) {
            float acc = dot_i8(NULL, A + (size_t)mi * K, W + (size_t)ni * K, K);
            C[(size_t)mi * N + (size_t)ni] = f32_to_bf16(acc * scales[ni]);
        }
    return 0;
}

/* kernels.c:658-737: argmax over bf16-rounded logits, ties -> lowest index. */
int oracle_linear_w8a16_bf16_argmax(size_t N, size_t K, const uint16_t *A, const int8_t *W,
                                    const float *scales, size_t *out_index, float *out_value) {
    if (!A || !W || !scales || !out_index || !out_value) return -1;
    if (N == 0 || K == 0) return -5;
    size_t best = 0;
    float best_v = -INFINITY;
    for (size_t n = 0; n < N; n++) {
        float v = bf16_to_f32(f32_to_bf16(dot_i8(NULL, A, W + n * K, K) * scales[n]));
        if (v > best_v || (v == best_v && n < best)) {
            best_v = v;
            best = n;
        }
    }
    *out_index = best;
    *out_value = best_v;
    return 0;
}

/* kernels.c:1002-1087 */
int oracle_linear_w4a16_bf16(size_t M, size_t N, size_t K, const uint16_t *A, const uint8_t *W,
                             const float *scales, uint16_t *C) {
    if (!A || !W || !scales || !C) return -1;
    const size_t pk = (K + 1) / 2;
    #pragma omp parallel for collapse(2) schedule(static)
    for (long long mi = 0; mi < (long long)M; mi++)
        for (long long ni = 0; ni < (long long)N; ni++) {
            float acc = dot_i4(A + (size_t)mi * K, W + (size_t)ni * pk, K);
            C[(size_t)mi * N + (size_t)ni] = f32_to_bf16(acc * scales[ni]);
        }
    return 0;
}

/* kernels.c:1089-1157: fresh dot per group, acc = fma(block, s[g], acc). */
int oracle_linear_w4a16g_bf16(size_t M, size_t N, size_t K, size_t group_size, const uint16_t *A,
                              const uint8_t *W, const float *scales, uint16_t *C) {
    if (!A || !W || !scales || !C || group_size == 0 || (group_size & 1)) return -1;
    const size_t pk = (K + 1) / 2;
    const size_t G = (K + group_size - 1) / group_size;
    #pragma omp parallel for collapse(2) schedule(static)
    for (long long mi = 0; mi < (long long)M; mi++)
        for (long long ni = 0; ni < (long long)N; ni++) {
            const uint16_t *a = A + (size_t)mi * K;
            const uint8_t *w = W + (size_t)ni * pk;
            const float *s = scales + (size_t)ni * G;
            float acc = 0.0f;
            for (size_t g = 0; g < G; g++) {
                size_t k0 = g * group_size;
                size_t gk = K - k0 < group_size ? K - k0 : group_size;
                float block = dot_i4(a + k0, w + k0 / 2, gk);
#if ORACLE_PLANT == 3
                {
                    float p = block * s[g];
                    acc = acc + p;
                }
#else
                acc = fmaf(block, s[g], acc);
#endif
            }
            C[(size_t)mi * N + (size_t)ni] = f32_to_bf16(acc);
        }
    return 0;
}

/* kernels.c:1580-1596: out = bf16(silu(g) * u), silu(g) = g / (1 + expf(-g)),
 * expf from the C library as in the reference build. */
static inline uint16_t swiglu_f32(float g, float u) {
#if ORACLE_PLANT == 9
    float silu = g / (1.0f + expf(g));
#else
    float silu = g / (1.0f + expf(-g));
#endif
    return f32_to_bf16(silu * u);
}

static inline uint16_t swiglu_one(uint16_t g_bits, uint16_t u_bits) {
    return swiglu_f32(bf16_to_f32(g_bits), bf16_to_f32(u_bits));
}

int oracle_swiglu_bf16(const uint16_t *gate, const uint16_t *up, uint16_t *out, size_t n) {
    if (!gate || !up || !out) return -1;
    for (size_t i = 0; i < n; i++) out[i] = swiglu_one(gate[i], up[i]);
    return 0;
}

/* kernels.c:1598-1735: M = 1; gate row i and up row I+i of the packed int4
 * gate_up matrix (per-row scales), each rounded to bf16 like a linear output,
 * hidden[i] = bf16(silu(g) * u), then the W4 per-row linear of hidden with the
 * down matrix.  Both dots are the per-row int4 dot (kernels.c:1639-1640 and
 * 1679 use the same 8-row / single-row dot functions as
 * ekernel_linear_w4a16_bf16). */
int oracle_swiglu_w4a16_bf16(size_t H, size_t I, size_t K, const uint16_t *A, const uint8_t *gate_up_W,
                             const float *gate_up_scales, const uint8_t *down_W, const float *down_scales,
                             uint16_t *C, uint16_t *hidden) {
    if (!A || !gate_up_W || !gate_up_scales || !down_W || !down_scales || !C || !hidden) return -1;
    if (H == 0 || I == 0 || K == 0) return -5;
    const size_t gpk = (K + 1) / 2, dpk = (I + 1) / 2;
    #pragma omp parallel for schedule(static)
    for (long long ii = 0; ii < (long long)I; ii++) {
        const size_t i = (size_t)ii;
        float gs = dot_i4(A, gate_up_W + i * gpk, K) * gate_up_scales[i];
        float us = dot_i4(A, gate_up_W + (I + i) * gpk, K) * gate_up_scales[I + i];
#if ORACLE_PLANT == 8
        hidden[i] = swiglu_f32(gs, us);
#else
        hidden[i] = swiglu_one(f32_to_bf16(gs), f32_to_bf16(us));
#endif
    }
    #pragma omp parallel for schedule(static)
    for (long long hh = 0; hh < (long long)H; hh++) {
        const size_t h = (size_t)hh;
        C[h] = f32_to_bf16(dot_i4(hidden, down_W + h * dpk, I) * down_scales[h]);
    }
    return 0;
}

/* The C library's expf over an array (used to pin the device expf). */
void oracle_expf(const float *x, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = expf(x[i]);
}

/* bf16 helpers exported for the Python side of the oracle. */
void oracle_f32_to_bf16(const float *x, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = f32_to_bf16(x[i]);
}
