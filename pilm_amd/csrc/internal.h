// Shared host-side plumbing of the HIP libecpu: error reporting, the current
// stream, and validation of the device buffers an entry point is handed.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/ecpu_hip.h"

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

// Per-device scratch the GEMV split path uses for partial sums (grown on
// demand, kept until ecpu_shutdown / process exit).
float *scratch_floats(size_t n, int *rc, const char *fn);

}  // namespace pilm
