"""CPU restatement of the reference's attention step -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only to check or to time the CPU side.

The reference computes this step in torch on the CPU
(src/models/qwen3/attention.py:95-139, FullAttention.forward after q_norm /
k_norm / rope) over the paged cache of src/runtime/kvcache/physical_kv.py:
11-81.  It is restated here as the same sequence of torch CPU operations on
the same dtypes, so the roundings are torch's own: a bf16 bmm for the scores,
a bf16 product with the Python-float scale, softmax in fp32, the weights
cast to bf16, a bf16 bmm for P.V, and the bf16 sigmoid gate.

Pinned by tests/test_oracle_attention.py against what the mathematics fixes:
one position gives its value row (and the gate's product) exactly, equal
keys give the mean of the values, head h reads kv head h // rep, a query
row does not see positions after its own, permuting the physical blocks
with the block table changes nothing, and the result agrees with a float64
numpy attention within the bf16 roundings.
"""
from __future__ import annotations

import math

import torch


def write_rows(k_cache, v_cache, block_ids, positions, keys, values) -> None:
    """physical_kv.py:37-51 (write): row i of keys / values goes to block
    block_ids[positions[i] // block_size], slot positions[i] % block_size."""
    bs = k_cache.shape[1]
    for i, pos in enumerate(positions):
        b, off = block_ids[pos // bs], pos % bs
        k_cache[b, off] = keys[i]
        v_cache[b, off] = values[i]


def read_seq(k_cache, v_cache, block_ids, n_valid):
    """physical_kv.py:56-70 (read_seq): the sequence's rows in position order."""
    k = torch.cat([k_cache[b] for b in block_ids], dim=0)[:n_valid]
    v = torch.cat([v_cache[b] for b in block_ids], dim=0)[:n_valid]
    return k, v


def paged_attention(q, k_new, v_new, k_cache=None, v_cache=None, block_ids=None, cache_len=None, gate=None):
    """attention.py:95-139 from the cache write to the gated output (before o_proj).

    q [S, H, D], k_new / v_new [S, Hkv, D], k_cache / v_cache [NB, BS, Hkv, D]
    (bf16 CPU tensors; the caches receive the new rows at positions
    cache_len - S ..), block_ids a list, gate [S, H, D] or None.
    Returns out [S, H * D] bf16.
    """
    seq, n_heads, head_dim = q.shape
    n_kv = k_new.shape[1]
    if k_cache is not None:
        # :95-97 write the step's rows; :98-109 gather positions 0 .. cache_len - 1
        write_rows(k_cache, v_cache, block_ids, range(cache_len - seq, cache_len), k_new, v_new)
        needed = (cache_len + k_cache.shape[1] - 1) // k_cache.shape[1]
        full_k, full_v = read_seq(k_cache, v_cache, block_ids[:needed], cache_len)
    else:
        # :115-116 no cache: the step's own rows
        full_k, full_v = k_new, v_new
    kv_len = full_k.shape[0]
    if n_kv < n_heads:
        # :119-122 each kv head serves n_heads / n_kv consecutive query heads
        rep = n_heads // n_kv
        full_k = full_k.unsqueeze(2).expand(-1, -1, rep, -1).reshape(kv_len, n_heads, head_dim)
        full_v = full_v.unsqueeze(2).expand(-1, -1, rep, -1).reshape(kv_len, n_heads, head_dim)
    qt = q.transpose(0, 1)
    kt = full_k.transpose(0, 1)
    vt = full_v.transpose(0, 1)
    scale = 1.0 / math.sqrt(head_dim)
    scores = torch.bmm(qt, kt.transpose(1, 2)) * scale                      # :127-129
    # :131-134 causal mask (a no-op for one decode row)
    mask = torch.triu(torch.ones(seq, kv_len, dtype=torch.bool), diagonal=kv_len - seq + 1)
    scores = scores.masked_fill(mask.unsqueeze(0), float("-inf"))
    attn = torch.softmax(scores.to(torch.float32), dim=-1).to(vt.dtype)   # :136
    out = torch.bmm(attn, vt)                                               # :137
    out = out.transpose(0, 1).reshape(seq, -1)                              # :138
    if gate is not None:
        out = out * torch.sigmoid(gate.reshape(seq, -1))                    # :139
    return out
