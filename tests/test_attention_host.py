"""Host-side checks of pilm_amd.attention that need no GPU: arguments the
wrapper rejects before calling the library, and the cache class's
bookkeeping (physical_kv.py:71-81)."""
from __future__ import annotations

import pytest
import torch

from pilm_amd import attention as A


def _bf(*shape):
    return torch.zeros(*shape, dtype=torch.bfloat16)


def test_host_tensors_rejected():
    with pytest.raises(ValueError, match="GPU tensor"):
        A.paged_attention(_bf(1, 16, 128), _bf(1, 8, 128), _bf(1, 8, 128))


def test_wrong_dtype_rejected():
    with pytest.raises(ValueError):
        A._check_dev("q", torch.zeros(1, 16, 128, dtype=torch.float32))


def test_block_table_from_list_and_tensor():
    t = A._block_table([3, 1, 2], "cpu", 4, 3)
    assert t.dtype == torch.int32 and t.tolist() == [3, 1, 2]
    t2 = A._block_table(torch.tensor([5, 4], dtype=torch.int64), "cpu", 8, 2)
    assert t2.dtype == torch.int32 and t2.is_contiguous() and t2.tolist() == [5, 4]


def test_block_table_rejects_invalid_ids():
    """As the reference's cache indexing does (physical_kv.py, attention.py:
    98-112): an id outside the cache raises IndexError, as does a table too
    short for the positions; ids past the needed blocks are not looked at."""
    with pytest.raises(IndexError, match="out of bounds"):
        A._block_table([0, 4], "cpu", 4, 2)
    with pytest.raises(IndexError, match="out of bounds"):
        A._block_table([-1], "cpu", 4, 1)
    with pytest.raises(IndexError, match="needed"):
        A._block_table([0], "cpu", 4, 2)
    assert A._block_table([0, 1, 99], "cpu", 4, 2).tolist() == [0, 1, 99]


def test_cache_bookkeeping_without_gpu():
    # the bookkeeping mirrors physical_kv.py: used blocks, free, total bytes
    cache = A.PagedKVCache.__new__(A.PagedKVCache)
    cache.num_layers, cache.num_blocks, cache.block_size = 28, 64, 16
    cache.num_kv_heads, cache.head_dim, cache.dtype = 8, 128, torch.bfloat16
    cache.used = {1, 2, 3}
    cache.free_blocks([2, 7])
    assert cache.num_used_blocks() == 2
    assert cache.total_bytes() == 64 * 16 * 8 * 128 * 2 * 28 * 2


def test_non_bf16_cache_rejected():
    with pytest.raises(ValueError, match="bf16"):
        A.PagedKVCache(1, 4, 16, 8, 128, dtype=torch.float32, device="cpu")
