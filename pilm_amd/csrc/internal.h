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

// Integer value of environment variable `name` (tuning overrides), else dflt.
int env_int(const char *name, int dflt);

// Exact GEMV of the per-row formats (fmt 0 W8A32, 1 W8A16, 2 W4A16 per-row)
// for K a multiple of the 128-byte stripe and 16-byte aligned W and A;
// enqueued on `st`.
int run_rows(int fmt, size_t M, size_t N, size_t K, const void *A, const uint8_t *W, const float *S, void *C,
             hipStream_t st, const char *fn);

}  // namespace pilm
