// extern "C" entry points of the quantized matrix-product path plus the two
// other kernels bindings.py:_configure requires (ekernel_gemm,
// ekernel_swiglu_bf16).  Each entry point keeps the reference's signature
// and null-pointer rule (ECPU_ERR_PARAM), then checks that every buffer is
// device memory large enough for the descriptor's shape before anything is
// launched, so a wrong pointer or shape becomes an error code instead of a
// GPU memory fault.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdlib>

#include "internal.h"

namespace pilm {
int run_linear(int fmt, size_t M, size_t N, size_t K, const void *A, const uint8_t *W, const float *S,
               void *C, const char *fn);
enum : int { F_W8A32 = 0, F_W8A16 = 1, F_W4ROW = 2, F_W4G128 = 3, F_W4G32 = 4 };
}  // namespace pilm

using namespace pilm;

// 0: no checks beyond NULL, 1: device-memory check, 2 (default): device
// memory and allocation extent.
static int check_level() {
    static int lvl = -1;
    if (lvl < 0) {
        const char *v = getenv("PILM_HIP_CHECK");
        lvl = (v && *v) ? atoi(v) : 2;
    }
    return lvl;
}

static int check_buf(const void *p, size_t bytes, const char *what, const char *fn) {
    const int lvl = check_level();
    if (!p) return fail(ECPU_ERR_PARAM, "%s: %s is NULL", fn, what);
    if (lvl <= 0) return ECPU_OK;
    return check_device_buffer(p, lvl >= 2 ? bytes : 0, what, fn);
}

static bool mul_ok(size_t a, size_t b, size_t *out) { return !__builtin_mul_overflow(a, b, out); }

static int linear_common(int fmt, const ekernel_linear_w8a32_desc_t *desc, const void *A, const void *W,
                         const float *S, void *C, const char *fn) {
    if (!desc || !A || !W || !S || !C) return fail(ECPU_ERR_PARAM, "%s: NULL argument", fn);
    const size_t M = desc->M, N = desc->N, K = desc->K;
    const size_t lim = (size_t)1 << 31;
    if (M >= lim || N >= lim || K >= lim) return fail(ECPU_ERR_PARAM, "%s: M/N/K must be < 2^31", fn);
    const bool w8 = (fmt == F_W8A32 || fmt == F_W8A16);
    const size_t a_elt = (fmt == F_W8A32) ? 4 : 2;
    const size_t row_bytes = w8 ? K : (K + 1) / 2;
    const size_t group = (fmt == F_W4G128) ? 128 : (fmt == F_W4G32 ? 32 : 0);
    const size_t ncols_s = group ? (K + group - 1) / group : 1;
    size_t a_bytes, w_bytes, s_bytes, c_bytes, t;
    if (!mul_ok(M, K, &t) || !mul_ok(t, a_elt, &a_bytes) || !mul_ok(N, row_bytes, &w_bytes) ||
        !mul_ok(N, ncols_s, &t) || !mul_ok(t, 4, &s_bytes) || !mul_ok(M, N, &t) || !mul_ok(t, a_elt, &c_bytes))
        return fail(ECPU_ERR_PARAM, "%s: shape overflows size_t", fn);
    int rc;
    if ((rc = check_buf(A, a_bytes, "A", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(W, w_bytes, "W", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(S, s_bytes, "scales", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(C, c_bytes, "C", fn)) != ECPU_OK) return rc;
    return run_linear(fmt, M, N, K, A, (const uint8_t *)W, S, C, fn);
}

// ------------------------------------------------------------ f32 GEMM
// kernels.c:396-435: 8-lane FMA dot when !transpose_a && transpose_b (and the
// caller's isa is AVX2 or above), otherwise a sequential FMA loop.
__device__ __forceinline__ float hsum8_(const float l[8]) {
    return ((l[0] + l[4]) + (l[1] + l[5])) + ((l[2] + l[6]) + (l[3] + l[7]));
}

__global__ __launch_bounds__(256) void gemm_f32_kernel(const float *__restrict__ A, const float *__restrict__ B,
                                                       float *__restrict__ C, size_t M, size_t N, size_t K,
                                                       int ta, int tb, int lanes8) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= M * N) return;
    const size_t m = idx / N, n = idx % N;
    const size_t lda = ta ? M : K, ldb = tb ? K : N;
    float acc;
    if (lanes8) {
        const float *a = A + m * lda, *b = B + n * ldb;
        float l8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        size_t k = 0;
        for (; k + 8 <= K; k += 8)
            for (int l = 0; l < 8; ++l) l8[l] = __builtin_fmaf(a[k + l], b[k + l], l8[l]);
        acc = hsum8_(l8);
        for (; k < K; ++k) acc = __builtin_fmaf(a[k], b[k], acc);
    } else {
        acc = 0.0f;
        for (size_t k = 0; k < K; ++k) {
            const float av = ta ? A[k * lda + m] : A[m * lda + k];
            const float bv = tb ? B[n * ldb + k] : B[k * ldb + n];
            acc = __builtin_fmaf(av, bv, acc);
        }
    }
    C[idx] = acc;
}

// ------------------------------------------------------------ SwiGLU
// kernels.c:1580-1596: bf16(silu(g) * u) with silu(g) = g / (1 + exp(-g)).
// exp is evaluated in double and rounded once to float.
__global__ __launch_bounds__(256) void swiglu_bf16_kernel(const uint16_t *__restrict__ g,
                                                          const uint16_t *__restrict__ u,
                                                          uint16_t *__restrict__ out, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float gv = __uint_as_float((uint32_t)g[i] << 16);
    const float uv = __uint_as_float((uint32_t)u[i] << 16);
    const float e = (float)exp(-(double)gv);
    const float silu = gv / (1.0f + e);
    uint32_t b = __float_as_uint(silu * uv);
    b += 0x7FFFu + ((b >> 16) & 1u);
    out[i] = (uint16_t)(b >> 16);
}

extern "C" {

int ekernel_linear_w8a32(const ekernel_linear_w8a32_desc_t *desc, const float *A, const int8_t *W,
                         const float *scales, float *C, ekernel_isa_t isa) {
    (void)isa;
    return linear_common(F_W8A32, desc, A, W, scales, C, "ekernel_linear_w8a32");
}

int ekernel_linear_w8a16_bf16(const ekernel_linear_w8a32_desc_t *desc, const uint16_t *A, const int8_t *W,
                              const float *scales, uint16_t *C, ekernel_isa_t isa) {
    (void)isa;
    return linear_common(F_W8A16, desc, A, W, scales, C, "ekernel_linear_w8a16_bf16");
}

int ekernel_linear_w4a16_bf16(const ekernel_linear_w8a32_desc_t *desc, const uint16_t *A, const uint8_t *W,
                              const float *scales, uint16_t *C, ekernel_isa_t isa) {
    (void)isa;
    return linear_common(F_W4ROW, desc, A, W, scales, C, "ekernel_linear_w4a16_bf16");
}

int ekernel_linear_w4a16g32_bf16(const ekernel_linear_w8a32_desc_t *desc, const uint16_t *A, const uint8_t *W,
                                 const float *scales, uint16_t *C, ekernel_isa_t isa) {
    (void)isa;
    return linear_common(F_W4G32, desc, A, W, scales, C, "ekernel_linear_w4a16g32_bf16");
}

int ekernel_linear_w4a16g128_bf16(const ekernel_linear_w8a32_desc_t *desc, const uint16_t *A,
                                  const uint8_t *W, const float *scales, uint16_t *C, ekernel_isa_t isa) {
    (void)isa;
    return linear_common(F_W4G128, desc, A, W, scales, C, "ekernel_linear_w4a16g128_bf16");
}

int ekernel_gemm(const ekernel_gemm_desc_t *desc, const void *A, const void *B, void *C, ekernel_isa_t isa) {
    const char *fn = "ekernel_gemm";
    if (!desc || !A || !B || !C) return fail(ECPU_ERR_PARAM, "%s: NULL argument", fn);
    if (desc->a_prec != ECPU_PRECISION_F32 || desc->b_prec != ECPU_PRECISION_F32 ||
        desc->out_prec != ECPU_PRECISION_F32)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: only f32 is supported", fn);
    const size_t M = desc->M, N = desc->N, K = desc->K;
    size_t ab, bb, cb, t;
    if (!mul_ok(M, K, &t) || !mul_ok(t, 4, &ab) || !mul_ok(N, K, &t) || !mul_ok(t, 4, &bb) ||
        !mul_ok(M, N, &t) || !mul_ok(t, 4, &cb))
        return fail(ECPU_ERR_PARAM, "%s: shape overflows size_t", fn);
    int rc;
    if ((rc = check_buf(A, ab, "A", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(B, bb, "B", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(C, cb, "C", fn)) != ECPU_OK) return rc;
    if (M * N == 0) return ECPU_OK;
    const int lanes8 = !desc->transpose_a && desc->transpose_b && (int)isa >= (int)EKERNEL_ISA_AVX2;
    gemm_f32_kernel<<<(M * N + 255) / 256, 256, 0, current_stream()>>>(
        (const float *)A, (const float *)B, (float *)C, M, N, K, desc->transpose_a, desc->transpose_b, lanes8);
    return check_launch(fn);
}

int ekernel_swiglu_bf16(const uint16_t *gate, const uint16_t *up, uint16_t *out, size_t n) {
    const char *fn = "ekernel_swiglu_bf16";
    if (!gate || !up || !out) return fail(ECPU_ERR_PARAM, "%s: NULL argument", fn);
    if (n >= ((size_t)1 << 62)) return fail(ECPU_ERR_PARAM, "%s: n too large", fn);
    int rc;
    if ((rc = check_buf(gate, n * 2, "gate", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(up, n * 2, "up", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(out, n * 2, "out", fn)) != ECPU_OK) return rc;
    if (n == 0) return ECPU_OK;
    swiglu_bf16_kernel<<<(n + 255) / 256, 256, 0, current_stream()>>>(gate, up, out, n);
    return check_launch(fn);
}

}  // extern "C"
