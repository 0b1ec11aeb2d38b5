"""Portable seeded synthetic data for the quantized matrix-product path.

Every value is derived from a counter-based splitmix64 stream with integer
arithmetic and exact float64 operations only, so the same seed produces the
same bytes on any host, numpy version or device.  "Normal" activations use
the Irwin-Hall sum of 12 uniforms minus 6 (mean 0, variance 1), which needs
no transcendental functions.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """n outputs of splitmix64 at counters offset..offset+n-1 for this seed."""
    with np.errstate(over="ignore"):
        base = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) * _GOLDEN
        z = base + (np.arange(offset, offset + n, dtype=np.uint64) + np.uint64(1)) * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform01(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """float64 uniforms in [0, 1) with 53 random bits (exact)."""
    return (splitmix64(seed, n, offset) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def normal(seed: int, n: int) -> np.ndarray:
    """float64 approx-N(0,1) values (Irwin-Hall, 12 uniforms each)."""
    u = (splitmix64(seed, 12 * n) >> np.uint64(40)).astype(np.float64) * (2.0 ** -24)
    return u.reshape(n, 12).sum(axis=1) - 6.0


def randint(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    """int64 uniform integers in the closed range [lo, hi] (Lemire reduction)."""
    span = np.uint64(hi - lo + 1)
    r = (splitmix64(seed, n) >> np.uint64(32)) * span >> np.uint64(32)
    return r.astype(np.int64) + lo


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (nearest even), returned as uint16 bit patterns.

    Same rounding as the reference's f32_to_bf16 (kernels.c:19-25) for
    finite inputs.
    """
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    bits = bits + np.uint64(0x7FFF) + ((bits >> np.uint64(16)) & np.uint64(1))
    return ((bits >> np.uint64(16)) & np.uint64(0xFFFF)).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


# --- workload generators (shapes and distributions of the benchmark configs) ---

def activations_f32(seed: int, m: int, k: int) -> np.ndarray:
    return normal(seed, m * k).astype(np.float32).reshape(m, k)


def activations_bf16(seed: int, m: int, k: int) -> np.ndarray:
    """bf16 bit patterns of ~N(0,1) activations, shape [m, k]."""
    return f32_to_bf16_bits(activations_f32(seed, m, k)).reshape(m, k)


def weights_i8(seed: int, n: int, k: int) -> np.ndarray:
    """int8 weights uniform in [-127, 127], shape [n, k]."""
    return randint(seed, n * k, -127, 127).astype(np.int8).reshape(n, k)


def weights_i4_packed(seed: int, n: int, k: int) -> np.ndarray:
    """Packed int4 rows [n, ceil(k/2)]: both nibbles uniform in [0, 15]
    (they decode to [-8, 7]); for odd k the unused high nibble is zero."""
    pk = (k + 1) // 2
    w = randint(seed, n * pk, 0, 255).astype(np.uint8).reshape(n, pk)
    if k % 2:
        w[:, -1] &= 0x0F
    return w


def scales_uniform(seed: int, shape, lo: float = 0.001, hi: float = 0.02, fp16_round: bool = True) -> np.ndarray:
    """fp32 scales ~U(lo, hi); optionally rounded through fp16 (exact in fp32)."""
    n = int(np.prod(shape))
    s = lo + (hi - lo) * uniform01(seed, n)
    s = s.astype(np.float16) if fp16_round else s
    return s.astype(np.float32).reshape(shape)
