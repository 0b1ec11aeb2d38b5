"""Paged attention and the KV cache on the GPU.

Mirrors the two reference pieces the attention step of a decode / verify
token runs through:

* `PagedKVCache` -- src/runtime/kvcache/physical_kv.py:11-81
  (`PhysicalKVCache`): per layer one K and one V tensor of shape
  [num_blocks, block_size, n_kv_heads, head_dim], here in HBM; the block ids
  are owned by the caller's scheduler, as in the reference.
* `paged_attention` -- src/models/qwen3/attention.py:95-139, the step of
  FullAttention.forward between rope and o_proj: write the step's K/V rows
  into the cache, attend over positions 0 .. cache_len - 1 with the causal
  mask, gate.  It runs as two HIP kernels behind the C ABI entry point
  ekernel_paged_attention_bf16 (pilm_amd/csrc/attention.hip).

There is no CPU path: every function here takes device tensors and raises
if the HIP library is missing.
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch

from . import bindings as abi


def _check_dev(name: str, t: torch.Tensor) -> None:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor")
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16")


def _block_table(block_ids, device, num_blocks: int, needed: int) -> torch.Tensor:
    """int32 device table.  A host list is checked like the reference's
    indexing (IndexError for ids outside [0, num_blocks), and for a table
    shorter than the cache_len positions need); a device table is not read
    back -- the kernels clamp its ids into [0, num_blocks), so an invalid id
    reads and writes another block instead of faulting, and callers with
    device tables own their validity."""
    if isinstance(block_ids, torch.Tensor):
        t = block_ids.to(device=device, dtype=torch.int32)
    else:
        ids = [int(b) for b in block_ids]
        bad = [b for b in ids[:needed] if not 0 <= b < num_blocks]
        if bad:
            raise IndexError(f"block id {bad[0]} is out of bounds for a cache of {num_blocks} blocks")
        if len(ids) < needed:
            raise IndexError(f"{needed} blocks are needed for the positions, the table has {len(ids)}")
        t = torch.tensor(ids, dtype=torch.int32).to(device)
    return t.contiguous()


def paged_attention(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                    k_cache: Optional[torch.Tensor] = None, v_cache: Optional[torch.Tensor] = None,
                    block_ids=None, cache_len: Optional[int] = None,
                    gate: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Attention of one sequence's S new tokens (attention.py:95-139).

    q [S, H, D]; k_new, v_new [S, Hkv, D] (after k_norm / rope); k_cache,
    v_cache [num_blocks, block_size, Hkv, D]; block_ids the sequence's block
    table (list or int32 tensor) in position order; cache_len the tokens in
    the sequence once these S are in (the reference's positions[-1] + 1).
    The new rows are stored at positions cache_len - S .. cache_len - 1.
    Without a cache (k_cache None) the S rows attend to each other only.
    gate: [S, H, D] or a strided view of q_proj's output (last dim stride 1,
    consecutive heads `gate.stride(1)` apart); None for no gate.
    Returns out [S, H * D] bf16 (the input of o_proj).
    """
    for name, t in (("q", q), ("k_new", k_new), ("v_new", v_new)):
        _check_dev(name, t)
    if q.dim() != 3 or k_new.dim() != 3 or v_new.shape != k_new.shape:
        raise ValueError("q must be [S, H, D] and k_new, v_new [S, Hkv, D]")
    seq, n_heads, head_dim = q.shape
    if k_new.shape[0] != seq or k_new.shape[2] != head_dim:
        raise ValueError(f"k_new shape {tuple(k_new.shape)} does not match q {tuple(q.shape)}")
    n_kv = k_new.shape[1]
    q = q.contiguous()
    k_new = k_new.contiguous()
    v_new = v_new.contiguous()
    if k_cache is not None:
        _check_dev("k_cache", k_cache)
        _check_dev("v_cache", v_cache)
        if k_cache.shape != v_cache.shape or k_cache.dim() != 4 or k_cache.shape[2:] != (n_kv, head_dim):
            raise ValueError("caches must be [num_blocks, block_size, n_kv_heads, head_dim]")
        if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
            raise ValueError("caches must be contiguous")
        if cache_len is None:
            raise ValueError("cache_len is required with a cache")
        num_blocks, block_size = k_cache.shape[0], k_cache.shape[1]
        table = _block_table(block_ids, q.device, num_blocks, -(-int(cache_len) // block_size))
    else:
        cache_len = seq if cache_len is None else cache_len
        table = None
        num_blocks = block_size = 0
    gate_ptr, gate_stride = 0, 0
    if gate is not None:
        _check_dev("gate", gate)
        if gate.shape != (seq, n_heads, head_dim) or gate.stride(2) != 1 or \
                gate.stride(0) != n_heads * gate.stride(1):
            gate = gate.contiguous()
        gate_ptr, gate_stride = gate.data_ptr(), gate.stride(1)
    out = torch.empty((seq, n_heads * head_dim), dtype=torch.bfloat16, device=q.device)
    abi.set_stream(torch.cuda.current_stream(q.device).cuda_stream)
    rc = abi.paged_attention_bf16_ptr(
        q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(),
        k_cache.data_ptr() if k_cache is not None else 0, v_cache.data_ptr() if v_cache is not None else 0,
        table.data_ptr() if table is not None else 0, gate_ptr, out.data_ptr(),
        seq, n_heads, n_kv, head_dim, int(cache_len), block_size, num_blocks,
        table.numel() if table is not None else 0, gate_stride)
    if rc != 0:
        raise RuntimeError(f"ekernel_paged_attention_bf16 failed: rc={rc} ({abi.last_error()})")
    return out


class PagedKVCache:
    """physical_kv.py:11-81 with the blocks in HBM.

    k_cache[layer] / v_cache[layer]: [num_blocks, block_size, n_kv_heads,
    head_dim].  Block ids come from the caller's scheduler; `used` tracks the
    blocks written, as the reference's does."""

    def __init__(self, num_layers: int, num_blocks: int, block_size: int, num_kv_heads: int, head_dim: int,
                 dtype: torch.dtype = torch.bfloat16, device: str | torch.device = "cuda"):
        if dtype != torch.bfloat16:
            raise ValueError("the device attention kernels take bf16 caches")
        self.num_layers = num_layers
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        shape = (num_blocks, block_size, num_kv_heads, head_dim)
        self.k_cache: List[torch.Tensor] = [torch.empty(shape, dtype=dtype, device=device) for _ in range(num_layers)]
        self.v_cache: List[torch.Tensor] = [torch.empty(shape, dtype=dtype, device=device) for _ in range(num_layers)]
        self.used: set = set()

    def write(self, layer_idx: int, block_ids: Sequence[int], slot_offsets: Sequence[int],
              keys: torch.Tensor, values: torch.Tensor) -> None:
        """physical_kv.py:37-51: keys / values [n_slots, n_kv_heads, head_dim]."""
        if len(block_ids) != len(slot_offsets) or keys.shape[0] != len(block_ids):
            raise ValueError("one block id and slot offset per row")
        dev = self.k_cache[layer_idx].device
        b = torch.tensor(list(block_ids), dtype=torch.long, device=dev)
        o = torch.tensor(list(slot_offsets), dtype=torch.long, device=dev)
        self.k_cache[layer_idx][b, o] = keys.to(device=dev, dtype=self.dtype)
        self.v_cache[layer_idx][b, o] = values.to(device=dev, dtype=self.dtype)
        self.used.update(int(x) for x in block_ids)

    def read_block(self, layer_idx: int, block_id: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """physical_kv.py:53-54."""
        return self.k_cache[layer_idx][block_id], self.v_cache[layer_idx][block_id]

    def read_seq(self, layer_idx: int, block_ids: Sequence[int], n_valid: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """physical_kv.py:56-69: [n_valid, n_kv_heads, head_dim] K and V."""
        idx = torch.tensor(list(block_ids), dtype=torch.long, device=self.k_cache[layer_idx].device)
        k = self.k_cache[layer_idx].index_select(0, idx).flatten(0, 1)[:n_valid]
        v = self.v_cache[layer_idx].index_select(0, idx).flatten(0, 1)[:n_valid]
        return k, v

    def attend(self, layer_idx: int, block_ids, cache_len: int, q: torch.Tensor, k_new: torch.Tensor,
               v_new: torch.Tensor, gate: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The attention step of one sequence on this layer's blocks (the new
        rows are written at positions cache_len - S ..)."""
        kc = self.k_cache[layer_idx]
        table = _block_table(block_ids, kc.device, kc.shape[0], -(-int(cache_len) // kc.shape[1]))
        if not isinstance(block_ids, torch.Tensor):   # (a device table is not read back)
            needed = (int(cache_len) + self.block_size - 1) // self.block_size
            self.used.update(int(x) for x in list(block_ids)[:needed])
        return paged_attention(q, k_new, v_new, self.k_cache[layer_idx], self.v_cache[layer_idx], table,
                               cache_len, gate)

    def num_used_blocks(self) -> int:
        return len(self.used)

    def free_blocks(self, block_ids: Sequence[int]) -> None:
        for bid in block_ids:
            self.used.discard(bid)

    def total_bytes(self) -> int:
        """physical_kv.py:78-81."""
        per_layer = self.num_blocks * self.block_size * self.num_kv_heads * self.head_dim
        return per_layer * 2 * self.num_layers * 2
