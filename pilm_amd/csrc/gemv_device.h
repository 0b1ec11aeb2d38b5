// Device-side building blocks shared by the exact GEMV kernels of the HIP
// libecpu (gfx950): formats, bf16 helpers, the exact int4 decode, the
// reference's horizontal sum, and the wait-count helper.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace pilm {

enum Fmt : int { F_W8A32 = 0, F_W8A16 = 1, F_W4ROW = 2, F_W4G128 = 3, F_W4G32 = 4 };

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Activations are read through the constant address space: the address is the
// same for every lane of a wave, so each load becomes one s_load and the
// bf16 -> fp32 shifts run on the scalar unit.  The buffer is never written by
// these kernels (the scalar cache is not coherent with vector stores).
typedef __attribute__((address_space(4))) const uint32_t cu32;
typedef __attribute__((address_space(4))) const float cf32;
__device__ __forceinline__ const cu32 *as_const(const void *p) { return (const cu32 *)(uintptr_t)p; }

__device__ __forceinline__ float bf16_lo(uint32_t x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t x) { return __uint_as_float(x & 0xFFFF0000u); }

// kernels.c:19-25 (no NaN special case, like the reference).
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
    uint32_t b = __float_as_uint(x);
    b += 0x7FFFu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}

// kernels.c:56-63
__device__ __forceinline__ float hsum8(const float l[8]) {
    return ((l[0] + l[4]) + (l[1] + l[5])) + ((l[2] + l[6]) + (l[3] + l[7]));
}

// Eight nibbles (k = 0..7 of this dword, low nibble first) as exact fp16:
//   q[0] = (w0, w4)  q[1] = (w1, w5)  q[2] = (w2, w6)  q[3] = (w3, w7)
// XOR 0x8 turns the two's-complement nibble v into u = v + 8; 0x6400|u is the
// fp16 value 1024 + u, and 0x6400|(u << 4) is 1024 + 16u.  Subtracting 1032,
// or scaling by 1/16 and subtracting 72, yields v exactly.
// `magic` must hold 0x64006400; callers pass it through an opaque register so
// the compiler emits one v_and_or_b32 per nibble pair (mask in an SGPR,
// magic in a VGPR) instead of an and followed by an or with a literal.
__device__ __forceinline__ void dequant_w4(uint32_t x, uint32_t magic, h2 q[4]) {
    const uint32_t u = x ^ 0x88888888u;
    const uint32_t v = u >> 8;
    const h2 bias = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const h2 sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
    const h2 bias16 = {(_Float16)-72.0f, (_Float16)-72.0f};
    q[0] = __builtin_bit_cast(h2, (u & 0x000F000Fu) | magic) + bias;
    q[1] = __builtin_bit_cast(h2, (u & 0x00F000F0u) | magic) * sixteenth + bias16;
    q[2] = __builtin_bit_cast(h2, (v & 0x000F000Fu) | magic) + bias;
    q[3] = __builtin_bit_cast(h2, (v & 0x00F000F0u) | magic) * sixteenth + bias16;
}

__device__ __forceinline__ uint32_t opaque_magic() {
    uint32_t m = 0x64006400u;
    asm volatile("" : "+v"(m));
    return m;
}

// Wait until at most VM vector-memory operations of this wave are in flight.
// A wave's vector memory operations complete in issue order, so this
// guarantees that everything issued before the last VM operations is done.
template <int VM>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(VM >= 0 && VM < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((VM & 0xF) | (0x7 << 4) | (0xF << 8) | ((VM >> 4) << 14));
}

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kStripe = 128;        // bytes of each row per stripe: one full cache line
constexpr int kNT = 2;              // cache policy of the weight stream: non-temporal

}  // namespace pilm
