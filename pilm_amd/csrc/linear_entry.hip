// extern "C" entry points of the quantized matrix-product path (the five
// linear formats and the two fused epilogues, lm_head argmax and W4 SwiGLU)
// plus the two other kernels bindings.py:_configure requires (ekernel_gemm,
// ekernel_swiglu_bf16).  Each entry point keeps the reference's signature
// and null-pointer rule (ECPU_ERR_PARAM), then checks that every buffer is
// device memory large enough for the descriptor's shape before anything is
// launched, so a wrong pointer or shape becomes an error code instead of a
// GPU memory fault.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdlib>

#include "gemv_device.h"
#include "internal.h"

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

// ------------------------------------------------------------ norm + linear
static bool overlaps(const void *a, size_t an, const void *b, size_t bn) {
    if (!a || !b) return false;
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return x < y + bn && y < x + an;
}

extern "C" int ekernel_rmsnorm_linear_w4a16g128_bf16(const ekernel_norm_linear_desc_t *desc, const uint16_t *x,
                                                     const uint16_t *residual, const uint16_t *norm_weight,
                                                     uint16_t *residual_out, const uint8_t *W, const float *scales,
                                                     uint16_t *out) {
    static const char *fn = "ekernel_rmsnorm_linear_w4a16g128_bf16";
    if (!desc || !x || !norm_weight || !W || !scales || !out) return fail(ECPU_ERR_PARAM, "%s: NULL argument", fn);
    const size_t M = desc->rows, N = desc->N, K = desc->K;
    if (M == 0 || N == 0) return ECPU_OK;
    if (M != 1) return fail(ECPU_ERR_UNSUPPORTED, "%s: one activation row per call (rows = %zu)", fn, M);
    if (K == 0 || K % 256 || K > 16384)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: K = %zu (a multiple of 256 up to 16384)", fn, K);
    if (N >= ((size_t)1 << 31)) return fail(ECPU_ERR_PARAM, "%s: N must be < 2^31", fn);
    if (desc->swiglu && N % 16)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: SwiGLU needs N (gate + up rows) a multiple of 16, got %zu", fn, N);
    const uintptr_t al = (uintptr_t)x | (uintptr_t)residual | (uintptr_t)norm_weight | (uintptr_t)residual_out |
                         (uintptr_t)W;
    if ((al & 15) || ((uintptr_t)scales & 3))
        return fail(ECPU_ERR_UNSUPPORTED, "%s: x, residual, norm weight, residual_out and W must be 16-byte aligned",
                    fn);
    const size_t row = K * 2, n_out = desc->swiglu ? N / 2 : N;
    // every workgroup reads x and residual while workgroup 0 writes
    // residual_out and all write out
    if (overlaps(residual_out, row, x, row) || overlaps(residual_out, row, residual, row) ||
        overlaps(out, n_out * 2, x, row) || overlaps(out, n_out * 2, residual, row) ||
        overlaps(out, n_out * 2, residual_out, row))
        return fail(ECPU_ERR_PARAM, "%s: out / residual_out overlap the inputs", fn);
    int rc;
    if ((rc = check_buf(x, row, "x", fn)) != ECPU_OK) return rc;
    if (residual && (rc = check_buf(residual, row, "residual", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(norm_weight, row, "norm_weight", fn)) != ECPU_OK) return rc;
    if (residual_out && (rc = check_buf(residual_out, row, "residual_out", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(W, N * (K / 2), "W", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(scales, N * (K / 128) * 4, "scales", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(out, n_out * 2, "out", fn)) != ECPU_OK) return rc;
    rc = run_gq_norm(desc->swiglu != 0, N, K, x, residual, norm_weight, residual_out, desc->eps, W, scales, out,
                     current_stream());
    if (rc == ECPU_ERR_DEVICE) return fail(rc, "%s: raising the LDS limit of the GEMV kernel failed", fn);
    if (rc != ECPU_OK) return fail(rc, "%s: shape does not fit the kernel (N = %zu, K = %zu)", fn, N, K);
    return check_launch(fn);
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
    return run_swiglu_bf16(gate, up, out, n, current_stream(), fn);
}

int ekernel_linear_w8a16_bf16_argmax(const ekernel_linear_w8a32_desc_t *desc, const uint16_t *A, const int8_t *W,
                                     const float *scales, size_t *out_index, float *out_value, ekernel_isa_t isa) {
    const char *fn = "ekernel_linear_w8a16_bf16_argmax";
    (void)isa;
    if (!desc || !A || !W || !scales || !out_index || !out_value) return fail(ECPU_ERR_PARAM, "%s: NULL argument", fn);
    if (desc->M != 1 || desc->N == 0 || desc->K == 0)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: needs M == 1 and N, K > 0 (got M=%zu N=%zu K=%zu)", fn, desc->M,
                    desc->N, desc->K);
    const size_t N = desc->N, K = desc->K;
    const size_t lim = (size_t)1 << 31;
    if (N >= lim || K >= lim) return fail(ECPU_ERR_PARAM, "%s: N/K must be < 2^31", fn);
    size_t w_bytes;
    if (!mul_ok(N, K, &w_bytes)) return fail(ECPU_ERR_PARAM, "%s: shape overflows size_t", fn);
    int rc;
    if ((rc = check_buf(A, 2 * K, "A", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(W, w_bytes, "W", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(scales, 4 * N, "scales", fn)) != ECPU_OK) return rc;
    // out_index / out_value may each be host memory (the reference's ctypes
    // byref; the call then waits for the result) or device memory (written
    // by the kernel; the call returns without waiting).
    const bool idx_dev = is_device_pointer(out_index), val_dev = is_device_pointer(out_value);
    if (idx_dev && (rc = check_buf(out_index, sizeof(size_t), "out_index", fn)) != ECPU_OK) return rc;
    if (val_dev && (rc = check_buf(out_value, sizeof(float), "out_value", fn)) != ECPU_OK) return rc;
    return run_linear_argmax_w8a16(N, K, A, (const uint8_t *)W, scales, out_index, out_value, idx_dev, val_dev, fn);
}

int ekernel_linear_w8a16_bf16_argmax_noalloc(const ekernel_linear_w8a32_desc_t *desc, const uint16_t *A,
                                             const int8_t *W, const float *scales, size_t *out_index,
                                             float *out_value, ekernel_isa_t isa) {
    const char *fn = "ekernel_linear_w8a16_bf16_argmax_noalloc";
    (void)isa;
    if (!desc || !A || !W || !scales || !out_index || !out_value) return fail(ECPU_ERR_PARAM, "%s: NULL argument", fn);
    if (desc->M != 1 || desc->N == 0 || desc->K == 0)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: needs M == 1 and N, K > 0 (got M=%zu N=%zu K=%zu)", fn, desc->M,
                    desc->N, desc->K);
    const size_t N = desc->N, K = desc->K;
    if (N > kStaticArgmaxMaxN)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: N = %zu exceeds the %zu logits its static scratch holds", fn, N,
                    kStaticArgmaxMaxN);
    if (K >= ((size_t)1 << 31)) return fail(ECPU_ERR_PARAM, "%s: K must be < 2^31", fn);
    size_t w_bytes;
    if (!mul_ok(N, K, &w_bytes)) return fail(ECPU_ERR_PARAM, "%s: shape overflows size_t", fn);
    int rc;
    if ((rc = check_buf(A, 2 * K, "A", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(W, w_bytes, "W", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(scales, 4 * N, "scales", fn)) != ECPU_OK) return rc;
    const bool idx_dev = is_device_pointer(out_index), val_dev = is_device_pointer(out_value);
    if (idx_dev && (rc = check_buf(out_index, sizeof(size_t), "out_index", fn)) != ECPU_OK) return rc;
    if (val_dev && (rc = check_buf(out_value, sizeof(float), "out_value", fn)) != ECPU_OK) return rc;
    return run_linear_argmax_w8a16_static(N, K, A, (const uint8_t *)W, scales, out_index, out_value, idx_dev, val_dev,
                                          fn);
}

int ekernel_swiglu_w4a16_bf16(const ekernel_w4a16_swiglu_desc_t *desc, const uint16_t *A, const uint8_t *gate_up_W,
                              const float *gate_up_scales, const uint8_t *down_W, const float *down_scales,
                              uint16_t *C, ekernel_isa_t isa) {
    const char *fn = "ekernel_swiglu_w4a16_bf16";
    (void)isa;
    if (!desc || !A || !gate_up_W || !gate_up_scales || !down_W || !down_scales || !C)
        return fail(ECPU_ERR_PARAM, "%s: NULL argument", fn);
    if (desc->M != 1 || desc->hidden_size == 0 || desc->intermediate_size == 0 || desc->gate_up_in_features == 0 ||
        desc->down_in_features != desc->intermediate_size)
        return fail(ECPU_ERR_UNSUPPORTED,
                    "%s: needs M == 1, nonzero sizes and down_in_features == intermediate_size "
                    "(got M=%zu hidden=%zu intermediate=%zu gate_up_in=%zu down_in=%zu)",
                    fn, desc->M, desc->hidden_size, desc->intermediate_size, desc->gate_up_in_features,
                    desc->down_in_features);
    const size_t H = desc->hidden_size, I = desc->intermediate_size, K = desc->gate_up_in_features;
    if (H >= ((size_t)1 << 31) || I >= ((size_t)1 << 30) || K >= ((size_t)1 << 31))
        return fail(ECPU_ERR_PARAM, "%s: hidden/gate_up_in must be < 2^31, intermediate < 2^30", fn);
    size_t gu_bytes, d_bytes;
    if (!mul_ok(2 * I, (K + 1) / 2, &gu_bytes) || !mul_ok(H, (I + 1) / 2, &d_bytes))
        return fail(ECPU_ERR_PARAM, "%s: shape overflows size_t", fn);
    int rc;
    if ((rc = check_buf(A, 2 * K, "A", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(gate_up_W, gu_bytes, "gate_up_W", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(gate_up_scales, 8 * I, "gate_up_scales", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(down_W, d_bytes, "down_W", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(down_scales, 4 * H, "down_scales", fn)) != ECPU_OK) return rc;
    if ((rc = check_buf(C, 2 * H, "C", fn)) != ECPU_OK) return rc;
    return run_swiglu_w4(H, I, K, A, gate_up_W, gate_up_scales, down_W, down_scales, C, fn);
}

}  // extern "C"
