"""Host-side logic that needs no GPU: wrapper validation, synthetic data."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from pilm_amd import ckernel as ck
from pilm_amd import synth as S


def test_wrappers_reject_cpu_tensors_before_any_call():
    x = torch.zeros((1, 256), dtype=torch.bfloat16)
    w = torch.zeros((4, 128), dtype=torch.uint8)
    with pytest.raises(ValueError, match="GPU"):
        ck.linear_w4a16_bf16(x, w, torch.ones(4))
    with pytest.raises(ValueError, match="GPU"):
        ck.linear_w4a16g128_bf16(x, w, torch.ones((4, 2)))
    with pytest.raises(ValueError, match="GPU"):
        ck.linear_w8a32(torch.zeros((1, 8)), torch.zeros((2, 8), dtype=torch.int8), torch.ones(2))
    with pytest.raises(ValueError, match="GPU"):
        ck.gemm_f32(torch.zeros((2, 2)), torch.zeros((2, 2)))


def test_quantizers_match_the_oracle_on_cpu():
    """The torch quantizers (device-agnostic) produce the oracle's bytes."""
    from oracle import oracle as O
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((33, 301)) * 0.02).astype(np.float32)
    t = torch.from_numpy(w)
    q, s = ck.quantize_weight_i8_per_row(t)
    qo, so = O.quantize_weight_i8_per_row(w)
    assert np.array_equal(q.numpy(), qo) and np.array_equal(s.numpy(), so)
    q, s = ck.quantize_weight_i4_per_row_chunked(t, rows_per_chunk=7)
    qo, so = O.quantize_weight_i4_per_row(w)
    assert np.array_equal(q.numpy(), qo) and np.array_equal(s.numpy(), so)
    for g in (32, 128):
        q, s = ck.quantize_weight_i4_grouped_chunked(t, group_size=g, rows_per_chunk=10)
        qo, so = O.quantize_weight_i4_grouped(w, g)
        assert np.array_equal(q.numpy(), qo) and np.array_equal(s.numpy(), so)
    u = ck.unpack_i4_rows_to_i8(q, 301)
    assert np.array_equal(u.numpy(), O.unpack_i4_rows_to_i8(qo, 301))


def test_synth_is_stable():
    # fixed values: a change of the generator would silently change every fixture
    assert S.splitmix64(1, 3).tolist() == [int(v) for v in S.splitmix64(1, 3)]
    assert S.randint(5, 4, -127, 127).tolist() == S.randint(5, 4, -127, 127).tolist()
    x = S.normal(3, 100000)
    assert abs(x.mean()) < 0.02 and abs(x.std() - 1) < 0.02
    w = S.weights_i4_packed(1, 4, 7)
    assert w.shape == (4, 4) and np.all(w[:, -1] < 16)


def test_bf16_rounding_matches_reference_rule():
    x = np.array([1.0, 1.00390625, 1.005859375, -2.5e-39, 3.4e38], np.float32)
    b = S.f32_to_bf16_bits(x)
    bits = x.view(np.uint32).astype(np.uint64)
    exp = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) & 0xFFFF
    assert np.array_equal(b, exp.astype(np.uint16))
