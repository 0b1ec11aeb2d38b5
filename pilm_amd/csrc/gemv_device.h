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

// expf as the reference's C library computes it (kernels.c:1592, 1647-1648
// call the C library's expf).  glibc's expf (since 2.27; from Arm's
// optimized-routines) evaluates exp(x) = 2^(k/32) * 2^(r/32) in double: a
// 32-entry table of 2^(i/32), a degree-3 polynomial in r, one rounding to
// float at the end.  Its x86-64 build for FMA hardware fuses the products
// marked below; that build is what the reference runs on.  The same steps in
// the same order give the same float for every input (|err| of the final
// result up to 0.502 ulp, i.e. not always the correctly rounded value, which
// is why a plain exp in double would disagree on a few inputs, e.g. x =
// -0x1.9cp-4).  Table entries: the bits of 2^(i/32) rounded to double, less
// i << 47 (the exponent is added back from k).
__device__ __forceinline__ float ref_expf(float x) {
#pragma clang fp contract(off)
    if (!(__builtin_fabsf(x) < 88.0f)) {
        if (x != x) return x + x;
        if (x == -__builtin_inff()) return 0.0f;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    constexpr uint64_t T[32] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);     // fused
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);   // fused
    const uint64_t t = T[ki % 32] + (ki << 47);
    const double s = __builtin_bit_cast(double, t);
    const double z = __builtin_fma(c0, r, c1);            // fused
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);                 // fused
    y = __builtin_fma(z, r2, y);                          // fused
    y = y * s;
    return (float)y;
}

// kernels.c:1588-1593, 1645-1649: bf16(silu(g) * u), silu(g) = g / (1 + expf(-g)).
__device__ __forceinline__ uint16_t swiglu_bf16_value(float g, float u) {
#pragma clang fp contract(off)
    const float silu = g / (1.0f + ref_expf(-g));
    return f32_to_bf16(silu * u);
}

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kStripe = 128;        // bytes of each row per stripe: one full cache line
constexpr int kNT = 2;              // cache policy of the weight stream: non-temporal

}  // namespace pilm
