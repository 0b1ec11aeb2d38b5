// The fused epilogues of the quantized matrix-product path:
//   - greedy decode's lm_head: W8A16 GEMV + argmax over the bf16 logits
//     (kernels.c:658-737, ekernel_linear_w8a16_bf16_argmax);
//   - the W4 SwiGLU MLP of one decode token: gate/up GEMV, bf16(silu(g) * u),
//     down GEMV (kernels.c:1598-1735, ekernel_swiglu_w4a16_bf16);
// plus the elementwise SwiGLU (kernels.c:1580-1596).  The GEMVs are the exact
// kernels of the unfused entry points, so every value is bit-identical to the
// reference.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <mutex>

#include "gemv_device.h"
#include "internal.h"

namespace pilm {
namespace {

constexpr int kArgThreads = 256;
constexpr int kArgStep = kArgThreads * 8;     // logits per workgroup per step (8 per lane)
constexpr int kArgMaxBlocks = 512;

// The reference scans n = 0..N-1 keeping (best_value, best_idx), starting
// from (-inf, 0), and takes v when v > best or (v == best and n < best_idx)
// (kernels.c:667-668, 694-698, 711-714).  That rule is a total order on
// (value, index) pairs -- larger value first, then lower index, +0 == -0 --
// under which NaN never wins (both comparisons are false), so the scan's
// result is the maximum of {(-inf, 0)} and the non-NaN pairs, whatever the
// order they are visited in.  The kernel reduces in that order.
__device__ __forceinline__ bool arg_better(float av, uint32_t an, float bv, uint32_t bn) {
    return av > bv || (av == bv && an < bn);
}

__device__ __forceinline__ void arg_take(float v, uint32_t n, float &bv, uint32_t &bn) {
    if (arg_better(v, n, bv, bn)) {
        bv = v;
        bn = n;
    }
}

__device__ __forceinline__ void arg_wave_reduce(float &bv, uint32_t &bn) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const uint32_t on = (uint32_t)__shfl_xor((int)bn, off);
        arg_take(ov, on, bv, bn);
    }
}

// Workgroup b reduces logits [b * per_block, min(N, (b+1) * per_block)) and
// parks (value bits, index) in part[2b..2b+1]; the last workgroup to finish
// (ticket) reduces the parked pairs and writes the result to result[0..1]
// and to whichever of out_index / out_value are device pointers (non-null).
// per_block is a multiple of 8 and y is 16-byte aligned.
__global__ __launch_bounds__(kArgThreads) void argmax_bf16_kernel(const uint16_t *__restrict__ y, uint32_t N,
                                                                  uint32_t per_block, uint32_t *part, int *ticket,
                                                                  uint32_t *result, size_t *out_index,
                                                                  float *out_value) {
    __shared__ float s_v[kArgThreads / 64];
    __shared__ uint32_t s_n[kArgThreads / 64];
    __shared__ int s_last;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float bv = -__builtin_inff();
    uint32_t bn = 0;
    const uint32_t lo = blockIdx.x * per_block;
    const uint32_t hi = min(N, lo + per_block);
    for (uint32_t base = lo + 8u * tid; base < hi; base += kArgStep) {
        if (base + 8 <= hi) {
            const u32x4 q = *(const u32x4 *)(y + base);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                arg_take(bf16_lo(q[j]), base + 2 * j, bv, bn);
                arg_take(bf16_hi(q[j]), base + 2 * j + 1, bv, bn);
            }
        } else {
            for (uint32_t n = base; n < hi; ++n) arg_take(__uint_as_float((uint32_t)y[n] << 16), n, bv, bn);
        }
    }
    arg_wave_reduce(bv, bn);
    if (lane == 0) {
        s_v[wave] = bv;
        s_n[wave] = bn;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kArgThreads / 64; ++w) arg_take(s_v[w], s_n[w], bv, bn);
        int last = 1;
        if (gridDim.x > 1) {
            // Agent-scope stores reach the device-coherent level; once they
            // have completed the thread takes a ticket.
            __hip_atomic_store(part + 2 * blockIdx.x, __float_as_uint(bv), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(part + 2 * blockIdx.x + 1, bn, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            wait_vmcnt<0>();
            const int t = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = (t == (int)gridDim.x - 1);
        }
        s_last = last;
        s_v[0] = bv;
        s_n[0] = bn;
    }
    __syncthreads();
    if (!s_last || wave != 0) return;
    if (gridDim.x > 1) {
        bv = -__builtin_inff();
        bn = 0;
        for (uint32_t b = lane; b < gridDim.x; b += 64) {
            const uint32_t v = __hip_atomic_load(part + 2 * b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint32_t n = __hip_atomic_load(part + 2 * b + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            arg_take(__uint_as_float(v), n, bv, bn);
        }
        arg_wave_reduce(bv, bn);
    } else {
        bv = s_v[0];
        bn = s_n[0];
    }
    if (lane == 0) {
        result[0] = __float_as_uint(bv);
        result[1] = bn;
        if (out_index) *out_index = (size_t)bn;
        if (out_value) *out_value = bv;
        if (gridDim.x > 1) __hip_atomic_store(ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

__global__ __launch_bounds__(256) void swiglu_bf16_kernel(const uint16_t *__restrict__ g,
                                                          const uint16_t *__restrict__ u,
                                                          uint16_t *__restrict__ out, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    out[i] = swiglu_bf16_value(__uint_as_float((uint32_t)g[i] << 16), __uint_as_float((uint32_t)u[i] << 16));
}

constexpr size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

__global__ void clear_int_kernel(int *p) {
    if (threadIdx.x == 0) *p = 0;
}

}  // namespace

int run_swiglu_bf16(const uint16_t *g, const uint16_t *u, uint16_t *out, size_t n, hipStream_t st, const char *fn) {
    if (n == 0) return ECPU_OK;
    swiglu_bf16_kernel<<<(n + 255) / 256, 256, 0, st>>>(g, u, out, n);
    return check_launch(fn);
}

namespace {

// The W8A16 GEMV into `logits`, then the argmax kernel with its parked pairs
// in `part`, its ticket and its result word pair; host outputs wait for the
// result.  clear_ticket: a one-thread kernel zeroes the ticket first.
int linear_argmax_core(size_t N, size_t K, const uint16_t *A, const uint8_t *W, const float *S, uint16_t *logits,
                       uint32_t *part, uint32_t *result, int *ticket, bool clear_ticket, size_t *out_index,
                       float *out_value, bool index_on_device, bool value_on_device, const char *fn) {
    hipStream_t st = current_stream();
    if (clear_ticket) clear_int_kernel<<<1, 64, 0, st>>>(ticket);
    // The GEMV into logits, then the argmax kernel over them; with
    // PILM_HIP_ARGMAX_EPILOGUE=1 the argmax as the GEMV's epilogue instead (no
    // logits written), where the stripe kernel takes the shape.  Measured at
    // the Qwen3 lm_head (151936 rows, MI355X): GEMV alone 54.3 / 117.8 us
    // (K 2048 / 4096), GEMV + argmax kernel 55.2 / 118.4 us, epilogue 61.0 /
    // 124.2 us -- every workgroup of the epilogue waits for its parked pair to
    // reach the device-coherent level before taking its ticket.
    hipEvent_t ev0 = prof_begin(st);
    int rc = env_int("PILM_HIP_ARGMAX_EPILOGUE", 0) != 0
                 ? run_rows_argmax(N, K, A, W, S, part, ticket, result, index_on_device ? out_index : nullptr,
                                   value_on_device ? out_value : nullptr, st)
                 : ECPU_ERR_UNSUPPORTED;
    if (rc == ECPU_OK) {
        rc = check_launch(fn);
        if (rc != ECPU_OK) return rc;
        prof_end(ev0, st, "w8a16_gemv_argmax", (double)N * (double)K + 4.0 * (double)N + 2.0 * (double)K,
                 2.0 * (double)N * (double)K);
    } else if (rc == ECPU_ERR_UNSUPPORTED) {
        prof_end(ev0, st, nullptr, 0.0, 0.0);
        rc = run_linear(F_W8A16, 1, N, K, A, W, S, logits, fn);
        if (rc != ECPU_OK) return rc;
        ev0 = prof_begin(st);
        const uint32_t nblk = (uint32_t)std::min<size_t>(kArgMaxBlocks, (N + kArgStep - 1) / kArgStep);
        const uint32_t per_block = (uint32_t)round_up((N + nblk - 1) / nblk, 8);
        argmax_bf16_kernel<<<nblk, kArgThreads, 0, st>>>(logits, (uint32_t)N, per_block, part, ticket, result,
                                                         index_on_device ? out_index : nullptr,
                                                         value_on_device ? out_value : nullptr);
        rc = check_launch(fn);
        if (rc != ECPU_OK) return rc;
        prof_end(ev0, st, "w8a16_argmax", 2.0 * (double)N, 0.0);
    } else {
        return fail(ECPU_ERR_DEVICE, "%s: raising the LDS limit of the GEMV kernel failed", fn);
    }
    if (index_on_device && value_on_device) return ECPU_OK;
    // Host outputs (the reference's binding passes ctypes byref): wait for the
    // result like the reference's synchronous call.
    uint32_t host[2] = {0, 0};
    if (hipMemcpyAsync(host, result, sizeof(host), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess) {
        const hipError_t e = hipGetLastError();
        return fail(ECPU_ERR_DEVICE, "%s: reading the argmax back failed: %s", fn, hipGetErrorString(e));
    }
    if (!index_on_device) *out_index = (size_t)host[1];
    if (!value_on_device) memcpy(out_value, &host[0], sizeof(float));
    return ECPU_OK;
}

// Scratch of the entry point that allocates nothing: the logits of up to
// kStaticArgmaxMaxN rows, the parked pairs, the result and the ticket, in one
// file-scope device array.  Each GPU holds its own copy (its address comes
// from hipGetSymbolAddress with that device current) for the whole process;
// calls that overlap in time on one GPU share it and race.
constexpr size_t kStaticLogitBytes = round_up(kStaticArgmaxMaxN * 2, 256);
constexpr size_t kStaticPartBytes = rows_argmax_tiles(kStaticArgmaxMaxN) * 8;
constexpr size_t kStaticBytes = kStaticLogitBytes + kStaticPartBytes + 256 + 256;
__device__ __align__(256) unsigned char scratch[kStaticBytes];

std::mutex g_static_mu;
void *g_static_ptr[64];

int static_scratch(void **p, const char *fn) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(ECPU_ERR_DEVICE, "%s: no current HIP device", fn);
    if (dev < 0 || dev >= 64) return fail(ECPU_ERR_DEVICE, "%s: device %d beyond the 64 this library tracks", fn, dev);
    std::lock_guard<std::mutex> lk(g_static_mu);
    if (!g_static_ptr[dev]) {
        void *q = nullptr;
        const hipError_t e = hipGetSymbolAddress(&q, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !q) {
            (void)hipGetLastError();
            return fail(ECPU_ERR_DEVICE, "%s: hipGetSymbolAddress of the static scratch failed: %s", fn,
                        hipGetErrorString(e));
        }
        g_static_ptr[dev] = q;
    }
    *p = g_static_ptr[dev];
    return ECPU_OK;
}

}  // namespace

int run_linear_argmax_w8a16(size_t N, size_t K, const uint16_t *A, const uint8_t *W, const float *S,
                            size_t *out_index, float *out_value, bool index_on_device, bool value_on_device,
                            const char *fn) {
    hipStream_t st = current_stream();
    const size_t logit_bytes = round_up(N * 2, 256);
    const size_t part_bytes = round_up(std::max<size_t>(kArgMaxBlocks, rows_argmax_tiles(N)) * 8, 256);
    void *Y = nullptr;
    int rc = aux_scratch(logit_bytes + part_bytes + 256, &Y, fn);
    if (rc != ECPU_OK) return rc;
    float *P = nullptr;
    int *T = nullptr;
    // Ticket 4095 of the split-K set: the K-split GEMV takes ticket t for
    // tile t of grids below 256 tiles, and every kernel leaves its tickets
    // at zero, so calls ordered on one stream never share a live ticket.
    rc = split_scratch(st, 0, 4096, &P, &T, fn);
    if (rc != ECPU_OK) return rc;
    return linear_argmax_core(N, K, A, W, S, (uint16_t *)Y, (uint32_t *)((char *)Y + logit_bytes),
                              (uint32_t *)((char *)Y + logit_bytes + part_bytes), T + 4095, false, out_index,
                              out_value, index_on_device, value_on_device, fn);
}

int run_linear_argmax_w8a16_static(size_t N, size_t K, const uint16_t *A, const uint8_t *W, const float *S,
                                   size_t *out_index, float *out_value, bool index_on_device, bool value_on_device,
                                   const char *fn) {
    if (N > kStaticArgmaxMaxN)
        return fail(ECPU_ERR_UNSUPPORTED, "%s: N = %zu exceeds the static scratch's %zu logits", fn, N,
                    kStaticArgmaxMaxN);
    void *base = nullptr;
    const int rc = static_scratch(&base, fn);
    if (rc != ECPU_OK) return rc;
    char *b = (char *)base;
    return linear_argmax_core(N, K, A, W, S, (uint16_t *)b, (uint32_t *)(b + kStaticLogitBytes),
                              (uint32_t *)(b + kStaticLogitBytes + kStaticPartBytes),
                              (int *)(b + kStaticLogitBytes + kStaticPartBytes + 256), true, out_index, out_value,
                              index_on_device, value_on_device, fn);
}

int run_swiglu_w4(size_t H, size_t I, size_t K, const uint16_t *A, const uint8_t *Wgu, const float *Sgu,
                  const uint8_t *Wd, const float *Sd, uint16_t *C, const char *fn) {
    hipStream_t st = current_stream();
    const size_t hidden_bytes = round_up(I * 2, 256);
    void *Y = nullptr;
    int rc = aux_scratch(hidden_bytes + round_up(4 * I, 256), &Y, fn);
    if (rc != ECPU_OK) return rc;
    uint16_t *hidden = (uint16_t *)Y;

    hipEvent_t ev0 = prof_begin(st);
    rc = run_swiglu_gate_up(I, K, A, Wgu, Sgu, hidden, st);
    if (rc == ECPU_OK) {
        rc = check_launch(fn);
        if (rc != ECPU_OK) return rc;
        const double row_bytes = (double)((K + 1) / 2);
        prof_end(ev0, st, "w4a16_swiglu_gate_up", 2.0 * (double)I * (row_bytes + 4.0) + 2.0 * (double)K + 2.0 * (double)I,
                 4.0 * (double)I * (double)K);
    } else if (rc == ECPU_ERR_UNSUPPORTED) {
        // Shapes the stripe kernel does not take: the gate/up rows through the
        // W4 GEMV into bf16 [g | u], then the elementwise SwiGLU.
        prof_end(ev0, st, nullptr, 0.0, 0.0);   // the GEMV below is timed on its own
        uint16_t *gu = (uint16_t *)((char *)Y + hidden_bytes);
        rc = run_linear(F_W4ROW, 1, 2 * I, K, A, Wgu, Sgu, gu, fn);
        if (rc != ECPU_OK) return rc;
        rc = run_swiglu_bf16(gu, gu + I, hidden, I, st, fn);
        if (rc != ECPU_OK) return rc;
    } else if (rc == ECPU_ERR_DEVICE) {
        return fail(ECPU_ERR_DEVICE, "%s: raising the LDS limit of the SwiGLU kernel failed", fn);
    } else {
        return fail(rc, "%s: SwiGLU gate/up launch failed", fn);
    }
    return run_linear(F_W4ROW, 1, H, I, hidden, Wd, Sd, C, fn);
}

}  // namespace pilm
