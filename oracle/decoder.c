/* TEST INFRASTRUCTURE ONLY -- CPU restatement of the torch steps of piLM's
 * Qwen3 decoder layer, with torch's CPU roundings.
 *
 * piLM runs these steps with torch on the CPU (src/models/base/layers.py:
 * 101-195, src/models/qwen3/attention.py:82-139, src/models/qwen3/model.py:
 * 54-70, 108-127).  torch is a dependency the reference does not pin
 * (pyproject.toml declares none); this image has torch 2.10.0, whose CPU
 * kernels compute, for the operations those lines use:
 *   - sum / mean over a contiguous last dim (ATen cpu/SumKernel.cpp,
 *     cascade_sum): eight-float vectors, four accumulators over vectors
 *     v = 4r + k, rows folded through a cascade of levels of 16, then the
 *     accumulators in order, the leftover vectors into the first, the lanes
 *     into a scalar in order after the scalar tail; mean = sum / n;
 *   - softmax over the last dim (cpu/SoftMaxKernel.cpp, _vec_softmax_lastdim)
 *     with the AVX2 kernels: max; exp(x - max) by SLEEF's expf_u10; sum by
 *     vec::reduce_all over eight-float vectors (lane j takes j mod 8, folded
 *     ((0+4)+(2+6))+((1+5)+(3+7)); fewer than eight values in order);
 *     x * (1 / sum);
 *   - sigmoid and silu of bf16 tensors: 1 / (1 + e) and x / (1 + e) with
 *     e = expf_u10(-x), rounded to bf16;
 *   - bmm of bf16 tensors without oneDNN (BlasKernel.cpp): for q @ k^T each
 *     dot is a halving tree (i + D/2, then i + D/4, ...); for w @ v each dot
 *     runs four accumulators on j mod 4 with the tail on the first, folded
 *     in order; when S * L * D < 400 the small-matrix kernel sums both in
 *     plain order;
 *   - elementwise ops on bf16 tensors in fp32, rounded to bf16 once.
 * Each of these is checked against torch itself by tests/test_oracle_decoder.py
 * (same library, same settings as the fixture: AVX2 kernels, oneDNN off).
 *
 * Compiled with contraction off: every fmaf below is deliberate (they only
 * take exact bf16 x bf16 products, where an FMA equals a multiply and an add).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

static inline float bf(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline uint16_t to_bf(float x) {   /* round to nearest even (finite inputs) */
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);   /* quiet NaN */
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static inline float bfr(float x) { return bf(to_bf(x)); }

static inline float f_of_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* SLEEF expf_u10 (sleefsimdsp.c xexpf), as torch's Vectorized<float>::exp. */
float oracle_sleef_expf(float d) {
    const float q = rintf(d * 1.442695040888963407359924681001892137426645954152985934135449406931f);
    const int qi = (int)q;
    float s = fmaf(q, -0.693145751953125f, d);
    s = fmaf(q, -1.428606765330187045e-06f, s);
    float u = 0.000198527617612853646278381f;
    u = fmaf(u, s, 0.00139304355252534151077271f);
    u = fmaf(u, s, 0.00833336077630519866943359f);
    u = fmaf(u, s, 0.0416664853692054748535156f);
    u = fmaf(u, s, 0.166666671633720397949219f);
    u = fmaf(u, s, 0.5f);
    const float ss = s * s;
    u = 1.0f + fmaf(ss, u, s);
    const int q1 = qi >> 1;
    u = u * f_of_bits((uint32_t)(q1 + 127) << 23);
    u = u * f_of_bits((uint32_t)(qi - q1 + 127) << 23);
    if (d < -104.0f) u = 0.0f;
    if (d > 100.0f) u = INFINITY;
    return u;
}

void oracle_sleef_expf_n(const float *x, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = oracle_sleef_expf(x[i]);
}

/* torch's sum of a contiguous fp32 row of n >= 8 values. */
float oracle_torch_sum(const float *x, size_t n) {
    const size_t nvec = n / 8, size_ilp = nvec / 4;
    size_t clog = 0;
    while (((size_t)1 << clog) < size_ilp) ++clog;
    const size_t level_power = clog / 4 > 4 ? clog / 4 : 4;
    const size_t step = (size_t)1 << level_power, mask = step - 1;
    float part[4][8];
    for (int k = 0; k < 4; ++k) {
        for (int l = 0; l < 8; ++l) {
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            size_t r = 0;
            while (r + step <= size_ilp) {
                for (size_t j = 0; j < step; ++j, ++r) acc[0] = acc[0] + x[8 * (4 * r + k) + l];
                for (int j = 1; j < 4; ++j) {
                    acc[j] = acc[j] + acc[j - 1];
                    acc[j - 1] = 0.0f;
                    if ((r & (mask << (j * level_power))) != 0) break;
                }
            }
            for (; r < size_ilp; ++r) acc[0] = acc[0] + x[8 * (4 * r + k) + l];
            float a = acc[0];
            for (int j = 1; j < 4; ++j) a = a + acc[j];
            part[k][l] = a;
        }
    }
    for (size_t v = 4 * size_ilp; v < nvec; ++v)
        for (int l = 0; l < 8; ++l) part[0][l] = part[0][l] + x[8 * v + l];
    float fin = 0.0f;
    for (size_t i = 8 * nvec; i < n; ++i) fin = fin + x[i];
    for (int l = 0; l < 8; ++l) fin = fin + (((part[0][l] + part[1][l]) + part[2][l]) + part[3][l]);
    return fin;
}

/* GemmaRMSNorm of one row given as fp32 values (layers.py:130-147). */
static void gemma_norm(const float *h, size_t n, const uint16_t *w, float eps, uint16_t *out) {
    float *sq = (float *)malloc(n * sizeof(float));
    for (size_t i = 0; i < n; ++i) sq[i] = h[i] * h[i];
    const float sum = oracle_torch_sum(sq, n);
    free(sq);
    const float r = 1.0f / sqrtf(sum / (float)n + eps);
    for (size_t i = 0; i < n; ++i) {
        const float y = bfr(h[i] * r);
        const float wp = bfr(bf(w[i]) + 1.0f);
        out[i] = to_bf(wp * y);
    }
}

void oracle_rmsnorm_gemma_bf16(size_t rows, size_t n, float eps, const uint16_t *x, const uint16_t *res,
                               const uint16_t *w, uint16_t *out, uint16_t *res_out) {
    float *h = (float *)malloc(n * sizeof(float));
    for (size_t m = 0; m < rows; ++m) {
        for (size_t i = 0; i < n; ++i) {
            float v = bf(x[m * n + i]);
            if (res) {
                v = bfr(v + bf(res[m * n + i]));
                if (res_out) res_out[m * n + i] = to_bf(v);
            }
            h[i] = v;
        }
        gemma_norm(h, n, w, eps, out + m * n);
    }
    free(h);
}

/* attention.py:82-97 up to the cache write: q/k GemmaRMSNorm, apply_rope
 * (layers.py:150-195) with tables cos/sin [positions, rot/2], k and v stored
 * at position pos0 + s of the paged caches [blocks, bs, Hkv, D]. */
void oracle_qk_norm_rope_bf16(size_t S, size_t H, size_t Hkv, size_t D, size_t rot, size_t q_stride, size_t kv_stride,
                              size_t pos0, float eps, const uint16_t *qg, const uint16_t *k, const uint16_t *v,
                              const uint16_t *qw, const uint16_t *kw, const float *cos_t, const float *sin_t,
                              uint16_t *q_out, uint16_t *k_cache, uint16_t *v_cache, const int32_t *block_ids,
                              size_t block_size) {
    float *h = (float *)malloc(D * sizeof(float));
    uint16_t *nb = (uint16_t *)malloc(D * sizeof(uint16_t));
    const size_t nf = rot / 2;
    for (size_t s = 0; s < S; ++s) {
        const size_t pos = pos0 + s;
        for (size_t head = 0; head < H + Hkv; ++head) {
            const int is_q = head < H;
            const size_t hk = is_q ? head : head - H;
            const uint16_t *src = is_q ? qg + s * q_stride + hk * 2 * D : k + s * kv_stride + hk * D;
            for (size_t i = 0; i < D; ++i) h[i] = bf(src[i]);
            gemma_norm(h, D, is_q ? qw : kw, eps, nb);
            uint16_t *dst;
            if (is_q) {
                dst = q_out + (s * H + hk) * D;
            } else {
                const size_t row = (((size_t)block_ids[pos / block_size] * block_size + pos % block_size) * Hkv + hk) * D;
                dst = k_cache + row;
                memcpy(v_cache + row, v + s * kv_stride + hk * D, D * sizeof(uint16_t));
            }
            for (size_t i = 0; i < D; ++i) {
                float o = bf(nb[i]);
                if (i < rot) {
                    const size_t f = i < nf ? i : i - nf;
                    const float c = cos_t[pos * nf + f], sn = sin_t[pos * nf + f];
                    const float a = bf(nb[f]), b = bf(nb[f + nf]);
                    o = i < nf ? (a * c) - (b * sn) : (a * sn) + (b * c);
                }
                dst[i] = to_bf(o);
            }
        }
    }
    free(h);
    free(nb);
}

/* bmm dot of a q row with a k row (BlasKernel.cpp): halving tree, or plain
 * order in the small-matrix kernel. */
static float score_dot(const float *q, const float *kr, size_t D, int naive) {
    if (naive) {
        float acc = 0.0f;
        for (size_t i = 0; i < D; ++i) acc = acc + q[i] * kr[i];
        return acc;
    }
    float p[128];
    for (size_t i = 0; i < D / 2; ++i) p[i] = q[i] * kr[i] + q[i + D / 2] * kr[i + D / 2];
    for (size_t w = D / 4; w >= 1; w /= 2)
        for (size_t i = 0; i < w; ++i) p[i] = p[i] + p[i + w];
    return p[0];
}

/* attention.py:99-139 over the paged cache: see ekernel_attention_exact_bf16. */
void oracle_attention_exact_bf16(size_t S, size_t H, size_t Hkv, size_t D, size_t cache_len, size_t block_size,
                                 const int32_t *block_ids, const uint16_t *q, const uint16_t *k_cache,
                                 const uint16_t *v_cache, const uint16_t *gate, size_t gate_row_stride,
                                 size_t gate_head_stride, uint16_t *out) {
    const size_t rep = H / Hkv;
    const int naive = S * cache_len * D < 400;
    const float scale = (float)(1.0 / sqrt((double)D));
    float *x = (float *)malloc(cache_len * sizeof(float));
    float *qf = (float *)malloc(D * sizeof(float));
    float *kf = (float *)malloc(D * sizeof(float));
    for (size_t s = 0; s < S; ++s) {
        const size_t vis = cache_len - S + s + 1;
        for (size_t h = 0; h < H; ++h) {
            const size_t kh = h / rep;
            for (size_t i = 0; i < D; ++i) qf[i] = bf(q[(s * H + h) * D + i]);
            for (size_t j = 0; j < vis; ++j) {
                const size_t row = (((size_t)block_ids[j / block_size] * block_size + j % block_size) * Hkv + kh) * D;
                for (size_t i = 0; i < D; ++i) kf[i] = bf(k_cache[row + i]);
                x[j] = bfr(bfr(score_dot(qf, kf, D, naive)) * scale);
            }
            /* softmax over the whole row: masked positions are exp(-inf) = 0 */
            float mx = -INFINITY;
            for (size_t j = 0; j < vis; ++j) mx = x[j] > mx ? x[j] : mx;
            for (size_t j = 0; j < cache_len; ++j) x[j] = j < vis ? oracle_sleef_expf(x[j] - mx) : 0.0f;
            float sum;
            if (cache_len < 8) {
                sum = x[0];
                for (size_t j = 1; j < cache_len; ++j) sum = sum + x[j];
            } else {
                float a[8];
                for (int c = 0; c < 8; ++c) a[c] = x[c];
                for (size_t j = 8; j < cache_len; ++j) a[j % 8] = a[j % 8] + x[j];
                sum = ((a[0] + a[4]) + (a[2] + a[6])) + ((a[1] + a[5]) + (a[3] + a[7]));
            }
            const float inv = 1.0f / sum;
            for (size_t j = 0; j < cache_len; ++j) x[j] = bfr(x[j] * inv);
            /* P.V */
            for (size_t d = 0; d < D; ++d) {
                float o;
                if (naive) {
                    o = 0.0f;
                    for (size_t j = 0; j < cache_len; ++j) {
                        const size_t row = (((size_t)block_ids[j / block_size] * block_size + j % block_size) * Hkv + kh) * D;
                        o = o + x[j] * bf(v_cache[row + d]);
                    }
                } else {
                    float p[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                    const size_t main_len = cache_len / 4 * 4;
                    for (size_t j = 0; j < cache_len; ++j) {
                        if (j >= vis) continue;   /* weight 0: adds a zero */
                        const size_t row = (((size_t)block_ids[j / block_size] * block_size + j % block_size) * Hkv + kh) * D;
                        const float pr = x[j] * bf(v_cache[row + d]);
                        if (j < main_len) p[j % 4] = p[j % 4] + pr;
                        else p[0] = p[0] + pr;
                    }
                    o = ((p[0] + p[1]) + p[2]) + p[3];
                }
                o = bfr(o);
                if (gate) {
                    const float g = bf(gate[s * gate_row_stride + h * gate_head_stride + d]);
                    o = o * bfr(1.0f / (1.0f + oracle_sleef_expf(-g)));
                }
                out[(s * H + h) * D + d] = to_bf(o);
            }
        }
    }
    free(x);
    free(qf);
    free(kf);
}

void oracle_silu_mul_bf16(const uint16_t *g, const uint16_t *u, size_t rows, size_t n, size_t in_stride,
                          uint16_t *out) {
    for (size_t m = 0; m < rows; ++m)
        for (size_t i = 0; i < n; ++i) {
            const float gv = bf(g[m * in_stride + i]);
            const float sl = bfr(gv / (1.0f + oracle_sleef_expf(-gv)));
            out[m * n + i] = to_bf(sl * bf(u[m * in_stride + i]));
        }
}

void oracle_sigmoid_bf16(const uint16_t *x, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = to_bf(1.0f / (1.0f + oracle_sleef_expf(-bf(x[i]))));
}

void oracle_silu_bf16(const uint16_t *x, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float v = bf(x[i]);
        out[i] = to_bf(v / (1.0f + oracle_sleef_expf(-v)));
    }
}

/* softmax of fp32 rows [rows, n] as torch's CPU kernel (AVX2, eight lanes). */
void oracle_softmax_f32(const float *x, float *out, size_t rows, size_t n) {
    for (size_t m = 0; m < rows; ++m) {
        const float *r = x + m * n;
        float *o = out + m * n;
        float mx = -INFINITY;
        for (size_t j = 0; j < n; ++j) mx = r[j] > mx ? r[j] : mx;
        for (size_t j = 0; j < n; ++j) o[j] = oracle_sleef_expf(r[j] - mx);
        float sum;
        if (n < 8) {
            sum = o[0];
            for (size_t j = 1; j < n; ++j) sum = sum + o[j];
        } else {
            float a[8];
            for (int c = 0; c < 8; ++c) a[c] = o[c];
            for (size_t j = 8; j < n; ++j) a[j % 8] = a[j % 8] + o[j];
            sum = ((a[0] + a[4]) + (a[2] + a[6])) + ((a[1] + a[5]) + (a[3] + a[7]));
        }
        const float inv = 1.0f / sum;
        for (size_t j = 0; j < n; ++j) o[j] = o[j] * inv;
    }
}

/* argmax of bf16 logits: first index of the largest value. */
size_t oracle_argmax_bf16(const uint16_t *x, size_t n) {
    size_t bi = 0;
    float bv = -INFINITY;
    for (size_t i = 0; i < n; ++i) {
        const float v = bf(x[i]);
        if (v > bv) {
            bv = v;
            bi = i;
        }
    }
    return bi;
}
