"""Seeded synthetic decoder weights and prompts, bit-identical on any device.

A decoder's random-init weights are ~N(0, std) fp32 values derived from a
counter-based 32-bit hash evaluated with int64 torch operations whose every
intermediate stays below 2^63, so the same (seed, tensor id) produces the
same bits on the CPU and on the GPU.  The "normal" value is the Irwin-Hall
sum of four 16-bit uniforms, centred and scaled: an integer of magnitude
< 2^18 (exact in fp32) times one fp32 constant, a correctly rounded product
everywhere.  No transcendental function is involved.

Tensor ids enumerate a decoder's weights in a fixed order (`tensor_ids`), so
a test can regenerate any single tensor without the others.
"""
from __future__ import annotations

import math
from typing import Dict

import torch

_M32 = 0xFFFFFFFF
_M64 = (1 << 64) - 1
# standard deviation of the sum of four uniforms on {0..65535}
_IH4_SD = math.sqrt((65536.0 ** 2 - 1.0) / 3.0)


def _key(seed: int, tensor_id: int, stream: int) -> int:
    """A 32-bit stream key from (seed, tensor id, stream) on Python ints."""
    x = (seed * 0x9E3779B97F4A7C15 + tensor_id * 0xBF58476D1CE4E5B9 + stream * 0x94D049BB133111EB + 1) & _M64
    x ^= x >> 31
    x = (x * 0xD6E8FEB86659FD93) & _M64
    x ^= x >> 32
    return x & _M32


def _mix32(h: torch.Tensor) -> torch.Tensor:
    """32-bit avalanche on int64 tensors holding values in [0, 2^32); both
    multipliers are below 2^31, so no product reaches 2^63."""
    h = h ^ (h >> 16)
    h = (h * 0x7FEB352D) & _M32
    h = h ^ (h >> 15)
    h = (h * 0x2C1B3C6D) & _M32
    return h ^ (h >> 16)


def hash32(seed: int, tensor_id: int, stream: int, offset: int, n: int, device) -> torch.Tensor:
    idx = torch.arange(offset, offset + n, dtype=torch.int64, device=device)
    return _mix32((idx + _key(seed, tensor_id, stream)) & _M32)


def normal_f32(seed: int, tensor_id: int, shape, std: float = 0.02, device="cpu",
               chunk: int = 1 << 24) -> torch.Tensor:
    """fp32 tensor of the given shape, ~N(0, std), in row-major element order."""
    n = int(math.prod(shape))
    out = torch.empty(n, dtype=torch.float32, device=device)
    c = torch.tensor(std / _IH4_SD, dtype=torch.float32, device=device)
    for off in range(0, n, chunk):
        m = min(chunk, n - off)
        h1 = hash32(seed, tensor_id, 1, off, m, device)
        h2 = hash32(seed, tensor_id, 2, off, m, device)
        s = (h1 & 0xFFFF) + (h1 >> 16) + (h2 & 0xFFFF) + (h2 >> 16) - 131070
        out[off:off + m] = s.to(torch.float32) * c
        del h1, h2, s
    return out.reshape(shape)


def token_ids(seed: int, n: int, vocab: int, stream_id: int = 1_000_000) -> torch.Tensor:
    """n uniform token ids in [0, vocab) (multiply-shift reduction)."""
    h = hash32(seed, stream_id, 1, 0, n, "cpu")
    return ((h * vocab) >> 32).to(torch.int64)


def tensor_ids(num_layers: int) -> Dict[str, int]:
    """Fixed enumeration of a decoder's weight tensors (names follow piLM's
    Qwen3Model module tree, src/models/qwen3/model.py:10-127)."""
    ids = {"embed_tokens": 0}
    per_layer = ("input_layernorm", "post_attention_layernorm", "self_attn.q_proj", "self_attn.k_proj",
                 "self_attn.v_proj", "self_attn.o_proj", "self_attn.q_norm", "self_attn.k_norm",
                 "mlp.gate", "mlp.up", "mlp.down")
    for i in range(num_layers):
        for j, name in enumerate(per_layer):
            ids[f"layers.{i}.{name}"] = 1 + 16 * i + j
    ids["norm"] = 1 + 16 * num_layers
    ids["lm_head"] = 2 + 16 * num_layers
    return ids
