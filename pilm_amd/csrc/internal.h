// Shared host-side plumbing of the HIP libecpu: error reporting, the current
// stream, and validation of the device buffers an entry point is handed.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "ecpu_hip.h"

namespace pilm {

// Records a message for ecpu_last_error() and returns rc.
int fail(int rc, const char *fmt, ...);

hipStream_t current_stream();

// ECPU_OK when [ptr, ptr + bytes) lies inside one device allocation of the
// current device; otherwise ECPU_ERR_PARAM with a message naming `what`.
// bytes == 0 accepts any non-null pointer.
int check_device_buffer(const void *ptr, size_t bytes, const char *what, const char *fn);

// ECPU_OK after a launch, ECPU_ERR_DEVICE with the HIP error text otherwise.
int check_launch(const char *fn);

// Scratch for the K-split GEMV path, one set per device: `nfloat`
// floats of per-group block sums and `nticket` ints of per-tile tickets that
// are zero whenever no kernel is running.  Grown on demand with hipMalloc;
// an outgrown set is retired, not freed, until ecpu_shutdown(), so a HIP
// graph that captured it stays valid.  Calls that overlap in time on one
// device (different streams) must not both take the split path.
int split_scratch(hipStream_t stream, size_t nfloat, size_t nticket, float **P, int **T, const char *fn);

// Per-device buffer of at least `bytes` for the matrix-core path's converted
// activations; same growth, retirement and sharing rules as split_scratch.
int act_scratch(size_t bytes, void **X, const char *fn);

// Dequant-GEMM on the matrix cores for M >= mfma_min_m() (env
// PILM_HIP_MFMA_MIN_M, default 64; 0 keeps every M on the exact kernels)
// when mfma_supports(): K a multiple of 64, 16-byte aligned A and W.
// Outputs are within 1e-2 (in practice ~1e-3) of the reference, not
// bit-identical.
int mfma_min_m();
bool mfma_supports(size_t K, const void *A, const uint8_t *W);
int run_mfma(int fmt, size_t M, size_t N, size_t K, const void *A, const uint8_t *W, const float *S, void *C,
             hipStream_t st, const char *fn);

// Per-call timing of ecpu_hip_profile_begin/end: prof_begin records a start
// event on `st` when profiling is on (else returns nullptr); prof_end records
// the stop event and files the pair under `family` with its algorithmic bytes
// and flops (nothing when ev0 is nullptr; family nullptr drops the start
// event).
hipEvent_t prof_begin(hipStream_t st);
void prof_end(hipEvent_t ev0, hipStream_t st, const char *family, double bytes, double flops);

// Per-device buffer of at least `bytes` for the fused entry points'
// intermediates (logits, SwiGLU hidden row); same growth, retirement and
// sharing rules as split_scratch.
int aux_scratch(size_t bytes, void **Y, const char *fn);

// True when p is device memory of the current HIP runtime (clears any error
// the query leaves).
bool is_device_pointer(const void *p);

// Integer value of environment variable `name` (tuning overrides), else dflt.
int env_int(const char *name, int dflt);

// Exact GEMV of the per-row formats (fmt 0 W8A32, 1 W8A16, 2 W4A16 per-row)
// for K a multiple of the 128-byte stripe and 16-byte aligned W and A;
// enqueued on `st`.
int run_rows(int fmt, size_t M, size_t N, size_t K, const void *A, const uint8_t *W, const float *S, void *C,
             hipStream_t st, const char *fn);

// Exact GEMV of the group formats (3 W4A16 g128, 4 g32) with 16-row tiles
// and K divided among up to four waves per tile, for K a multiple of 256 and
// 16-byte aligned A and W; ECPU_ERR_UNSUPPORTED when LDS cannot hold a row.
int run_group_quad(int fmt, size_t M, size_t N, size_t K, const void *A, const uint8_t *W, const float *S, void *C,
                   hipStream_t st, const char *fn);

// W8A16 GEMV of one activation row with the greedy argmax epilogue
// (kernels.c:658-737), no logits written: part holds 2 * rows_argmax_tiles(N)
// words, the ticket must be zero (it is left at zero); ECPU_ERR_UNSUPPORTED
// when the shape or alignment does not suit the kernel (nothing launched).
// Workgroups of the argmax GEMV: 64-row tiles, or at most 512 smaller ones.
constexpr size_t rows_argmax_tiles(size_t N) { return (N + 63) / 64 > 512 ? (N + 63) / 64 : 512; }
int run_rows_argmax(size_t N, size_t K, const uint16_t *A, const uint8_t *W, const float *S, uint32_t *part,
                    int *ticket, uint32_t *result, size_t *out_index, float *out_value, hipStream_t st);

// One activation row of W4A16 g128 through a GemmaRMSNorm prologue
// (h = x + res, res_out = h, a = norm(h)) computed by every workgroup, then
// the group-quad GEMV of a; with swiglu, W = [gate; up] (N/2 rows each) and
// C[i] = bf16(bf16(silu(gate_i)) * up_i).  K a multiple of 256; enqueued on st.
int run_gq_norm(bool swiglu, size_t N, size_t K, const uint16_t *x, const uint16_t *res, const uint16_t *norm_w,
                uint16_t *res_out, float eps, const uint8_t *W, const float *S, uint16_t *C, hipStream_t st);

// Fused W4 SwiGLU gate/up pass (one launch) for M = 1; ECPU_ERR_UNSUPPORTED
// when the shape or alignment does not suit the stripe kernel.
int run_swiglu_gate_up(size_t I, size_t K, const uint16_t *A, const uint8_t *W, const float *S, uint16_t *hidden,
                       hipStream_t st);

// Every linear format and M on the current stream (exact kernels; matrix
// cores for M >= mfma_min_m()).
int run_linear(int fmt, size_t M, size_t N, size_t K, const void *A, const uint8_t *W, const float *S, void *C,
               const char *fn);

// Elementwise bf16 SwiGLU of n elements on `st`.
int run_swiglu_bf16(const uint16_t *g, const uint16_t *u, uint16_t *out, size_t n, hipStream_t st, const char *fn);

// W8A16 GEMV of one row + argmax of its bf16 logits on the current stream.
// An output flagged *_on_device is written by the kernel (the call returns
// without waiting); the others are host memory, filled after the stream has
// been synchronized.
int run_linear_argmax_w8a16(size_t N, size_t K, const uint16_t *A, const uint8_t *W, const float *S,
                            size_t *out_index, float *out_value, bool index_on_device, bool value_on_device,
                            const char *fn);

// The same with every intermediate (logits, parked pairs, result, ticket) in
// a file-scope device array instead of allocated scratch: no allocation at
// all; N <= kStaticArgmaxMaxN (else ECPU_ERR_UNSUPPORTED); overlapping calls
// on one GPU race on the array.
constexpr size_t kStaticArgmaxMaxN = 262144;
int run_linear_argmax_w8a16_static(size_t N, size_t K, const uint16_t *A, const uint8_t *W, const float *S,
                                   size_t *out_index, float *out_value, bool index_on_device, bool value_on_device,
                                   const char *fn);

// The W4 SwiGLU MLP of one token: C[H] = down(bf16(silu(g) * u)) with g, u
// the first and second I rows of the gate/up GEMV over K inputs.
int run_swiglu_w4(size_t H, size_t I, size_t K, const uint16_t *A, const uint8_t *Wgu, const float *Sgu,
                  const uint8_t *Wd, const float *Sd, uint16_t *C, const char *fn);

}  // namespace pilm
