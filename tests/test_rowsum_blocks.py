"""The GemmaRMSNorm sum of squares in torch's CPU order (oracle/decoder.py
restates it; pilm_amd/csrc/cpu_order.h computes it on the device two ways):
32 chains over 8-float vectors, each chain a cascade of 16-vector blocks.
The device's workgroup version sums the blocks independently and replays
the cascade over the block sums (row_sumsq_blocks + wave_row_rsqrt_blocks);
this checks, in fp32 on the CPU, that the replay equals the serial chain
(chain_sumsq) bit for bit for every row length the kernels take
(n % 32 == 0, up to 16384), including the remainder blocks and the second
cascade level (n > 8192)."""
from __future__ import annotations

import numpy as np
import pytest

f32 = np.float32


def _chain_serial(x, n, t):
    k, l = t >> 3, t & 7
    nvec = n // 8
    size_ilp = nvec // 4
    clog = 0
    while (1 << clog) < size_ilp:
        clog += 1
    lp = max(4, clog // 4)
    step, mask = 1 << lp, (1 << lp) - 1
    acc = [f32(0)] * 4
    r = 0
    while r + step <= size_ilp:
        for _ in range(0, step, 16):
            for j in range(16):
                v = x[8 * (4 * (r + j) + k) + l]
                acc[0] = f32(acc[0] + f32(v * v))
            r += 16
        for j in range(1, 4):
            acc[j] = f32(acc[j] + acc[j - 1])
            acc[j - 1] = f32(0)
            if r & (mask << (j * lp)):
                break
    while r < size_ilp:
        v = x[8 * (4 * r + k) + l]
        acc[0] = f32(acc[0] + f32(v * v))
        r += 1
    a = acc[0]
    for j in range(1, 4):
        a = f32(a + acc[j])
    return a


def _chain_blocks(x, n, t):
    k, l = t >> 3, t & 7
    size_ilp = n // 32
    nblk, rem = size_ilp // 16, size_ilp % 16
    bs = []
    for b in range(nblk + (1 if rem else 0)):
        a = f32(0)
        for j in range(16 if b < nblk else rem):
            v = x[8 * (4 * (16 * b + j) + k) + l]
            a = f32(a + f32(v * v))
        bs.append(a)
    a1 = a2 = a3 = f32(0)
    for b in range(nblk):
        r = 16 * (b + 1)
        a1 = f32(a1 + bs[b])
        if (r & (15 << 4)) == 0:
            a2, a1 = f32(a2 + a1), f32(0)
            if (r & (15 << 8)) == 0:
                a3, a2 = f32(a3 + a2), f32(0)
    a0 = bs[nblk] if rem else f32(0)
    return f32(f32(f32(a0 + a1) + a2) + a3)


@pytest.mark.parametrize("n", [32, 256, 768, 2048, 4096, 5120, 8192, 12288, 16384])
def test_block_replay_equals_serial_chain(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * rng.choice([1e-3, 1.0, 30.0], n)).astype(np.float32)
    x = (x.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)    # bf16 values, as the kernels see
    for t in range(32):
        a, b = _chain_serial(x, n, t), _chain_blocks(x, n, t)
        assert a.view(np.uint32) == b.view(np.uint32), f"n={n} chain {t}: {a!r} vs {b!r}"
