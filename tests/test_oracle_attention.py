"""Pins the CPU restatement of the attention step (oracle/attention.py)
against what the mathematics fixes -- no GPU needed."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as OA


def _bf(x) -> torch.Tensor:
    return torch.as_tensor(x, dtype=torch.float32).to(torch.bfloat16)


def _case(seed, S, H, Hkv, D, L, BS=16, nb_extra=3):
    g = torch.Generator().manual_seed(seed)
    q = _bf(torch.randn(S, H, D, generator=g))
    k_new = _bf(torch.randn(S, Hkv, D, generator=g))
    v_new = _bf(torch.randn(S, Hkv, D, generator=g))
    nblk = (L + BS - 1) // BS
    NB = nblk + nb_extra
    kc = _bf(torch.randn(NB, BS, Hkv, D, generator=g))
    vc = _bf(torch.randn(NB, BS, Hkv, D, generator=g))
    ids = torch.randperm(NB, generator=g)[:nblk].tolist()
    return q, k_new, v_new, kc, vc, ids


def _f64_attention(q, k, v, causal_base):
    """Plain float64 attention: q [S,H,D], k/v [L,H,D] (already expanded)."""
    qn, kn, vn = (t.double().numpy() for t in (q, k, v))
    S, H, D = qn.shape
    out = np.zeros((S, H, D))
    for s in range(S):
        for h in range(H):
            sc = kn[: causal_base + s + 1, h] @ qn[s, h] / math.sqrt(D)
            w = np.exp(sc - sc.max())
            w /= w.sum()
            out[s, h] = w @ vn[: causal_base + s + 1, h]
    return out.reshape(S, H * D)


def test_single_position_returns_value_row():
    q, k, v, _, _, _ = _case(1, 1, 4, 2, 64, 1)
    out = OA.paged_attention(q, k, v)
    rep = 2
    expect = v.repeat_interleave(rep, dim=1).reshape(1, -1)
    assert torch.equal(out, expect)
    gate = _bf(torch.randn(1, 4, 64, generator=torch.Generator().manual_seed(5)))
    out_g = OA.paged_attention(q, k, v, gate=gate)
    sig = torch.sigmoid(gate.float()).to(torch.bfloat16).reshape(1, -1)
    assert torch.equal(out_g, (expect.float() * sig.float()).to(torch.bfloat16))


def test_equal_keys_give_mean_of_values():
    S, H, Hkv, D, L = 1, 2, 1, 64, 40
    q, k_new, v_new, kc, vc, ids = _case(2, S, H, Hkv, D, L)
    kc[:] = kc[0, 0]          # every cached key equals the new key
    k_new[:] = kc[0, 0]
    out = OA.paged_attention(q, k_new, v_new, kc, vc, ids, L).float()
    _, vfull = OA.read_seq(kc, vc, ids, L)
    mean = vfull.float().mean(0).reshape(1, -1).repeat(1, H)
    # each weight is bf16(1/40); the sum of 40 values is then ~ (1 + 2^-9) of the mean
    assert torch.allclose(out, mean, atol=2e-2, rtol=1e-2)


def test_gqa_head_mapping():
    S, H, Hkv, D, L = 1, 8, 2, 64, 20
    q, k_new, v_new, kc, vc, ids = _case(3, S, H, Hkv, D, L)
    for kvh in range(Hkv):   # constant value row per kv head
        vc[:, :, kvh] = float(kvh + 1)
        v_new[:, kvh] = float(kvh + 1)
    out = OA.paged_attention(q, k_new, v_new, kc, vc, ids, L).float().reshape(H, D)
    for h in range(H):
        assert torch.all(out[h] == float(h // (H // Hkv) + 1)), h


def test_causal_rows_ignore_later_positions():
    S, H, Hkv, D, L = 4, 4, 2, 64, 50
    q, k_new, v_new, kc, vc, ids = _case(4, S, H, Hkv, D, L)
    out = OA.paged_attention(q, k_new, v_new, kc.clone(), vc.clone(), ids, L)
    k2, v2 = k_new.clone(), v_new.clone()
    k2[2:] = _bf(torch.randn(2, Hkv, D))   # rows 0 and 1 must not see tokens 2 and 3
    v2[2:] = _bf(torch.randn(2, Hkv, D))
    out2 = OA.paged_attention(q, k2, v2, kc.clone(), vc.clone(), ids, L)
    assert torch.equal(out[:2], out2[:2])
    assert not torch.equal(out[2:], out2[2:])


def test_block_permutation_changes_nothing():
    S, H, Hkv, D, L, BS = 2, 4, 4, 128, 70, 16
    q, k_new, v_new, kc, vc, ids = _case(5, S, H, Hkv, D, L, BS)
    out = OA.paged_attention(q, k_new, v_new, kc.clone(), vc.clone(), ids, L)
    perm = torch.randperm(kc.shape[0], generator=torch.Generator().manual_seed(9))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(len(perm))
    kc2, vc2 = kc[perm].clone(), vc[perm].clone()       # block b now lives at inv[b]
    ids2 = [int(inv[b]) for b in ids]
    out2 = OA.paged_attention(q, k_new, v_new, kc2, vc2, ids2, L)
    assert torch.equal(out, out2)


def test_cache_receives_new_rows():
    S, H, Hkv, D, L, BS = 3, 2, 1, 64, 35, 16
    q, k_new, v_new, kc, vc, ids = _case(6, S, H, Hkv, D, L, BS)
    OA.paged_attention(q, k_new, v_new, kc, vc, ids, L)
    for i in range(S):
        pos = L - S + i
        assert torch.equal(kc[ids[pos // BS], pos % BS], k_new[i])
        assert torch.equal(vc[ids[pos // BS], pos % BS], v_new[i])


@pytest.mark.parametrize("S,H,Hkv,D,L", [(1, 16, 8, 128, 300), (5, 32, 8, 128, 97), (3, 4, 4, 64, 3),
                                         (2, 8, 1, 256, 130)])
def test_against_float64_attention(S, H, Hkv, D, L):
    q, k_new, v_new, kc, vc, ids = _case(7 + S, S, H, Hkv, D, L)
    out = OA.paged_attention(q, k_new, v_new, kc, vc, ids, L if L > S else S) if L > S else \
        OA.paged_attention(q, k_new, v_new)
    kf, vf = OA.read_seq(kc, vc, ids, L) if L > S else (k_new, v_new)
    rep = H // Hkv
    kf = kf.repeat_interleave(rep, dim=1)
    vf = vf.repeat_interleave(rep, dim=1)
    ref = _f64_attention(q, kf, vf, L - S)
    err = np.abs(out.float().numpy() - ref).max()
    assert err <= 3e-2 * np.abs(ref).max(), err
    # a dropped 1/sqrt(D) or a transposed operand is far outside that bound
    wrong = _f64_attention(q * math.sqrt(D), kf, vf, L - S)
    assert np.abs(out.float().numpy() - wrong).max() > 10 * err
