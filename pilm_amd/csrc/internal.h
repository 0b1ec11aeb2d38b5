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

}  // namespace pilm
