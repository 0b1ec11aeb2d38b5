"""GPU parity of the paged attention kernels against the attention oracle.

Calls go through the C ABI (pilm_amd.attention -> ctypes ->
ekernel_paged_attention_bf16).  The oracle runs the reference's torch CPU
operations; the kernels reproduce its roundings (bf16 scores, bf16 scaled
scores, fp32 softmax, bf16 weights, bf16 P.V, bf16 gate) but not its fp32
summation orders or its exp, so a score or weight that falls next to a bf16
rounding boundary can land one bf16 step away.  Tolerance, per call: at
least 98 % of the outputs bit-identical, and every output within 1e-2 of
the oracle's largest output magnitude (measured: >= 99 % identical, largest
error 0.23 % of it; a wrong mask, scale, head mapping or block lookup moves
outputs by far more).  The caches after the call must
hold the oracle's rows exactly (the new rows are copies).
"""
from __future__ import annotations

import sys

import pytest
import torch

from oracle import attention as OA
from pilm_amd import attention as A

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _bf(x) -> torch.Tensor:
    return torch.as_tensor(x, dtype=torch.float32).to(torch.bfloat16)


def _inputs(seed, S, H, Hkv, D, L, BS, cache=True, gate="none"):
    g = torch.Generator().manual_seed(seed)
    q = _bf(torch.randn(S, H, D, generator=g))
    k_new = _bf(torch.randn(S, Hkv, D, generator=g))
    v_new = _bf(torch.randn(S, Hkv, D, generator=g))
    kc = vc = ids = None
    if cache:
        nblk = (L + BS - 1) // BS
        NB = nblk + 5
        kc = _bf(torch.randn(NB, BS, Hkv, D, generator=g))
        vc = _bf(torch.randn(NB, BS, Hkv, D, generator=g))
        ids = torch.randperm(NB, generator=g)[:nblk].tolist()
    qg = None
    if gate != "none":
        qg = _bf(torch.randn(S, H, 2 * D, generator=g))   # q_proj's output: query | gate per head
    return q, k_new, v_new, kc, vc, ids, qg


def _run_both(dev, S, H, Hkv, D, L, BS=16, cache=True, gate="none", seed=0):
    q, k_new, v_new, kc, vc, ids, qg = _inputs(seed, S, H, Hkv, D, L, BS, cache, gate)
    gate_cpu = qg[:, :, D:] if qg is not None else None
    ref_kc = kc.clone() if kc is not None else None
    ref_vc = vc.clone() if vc is not None else None
    ref = OA.paged_attention(q, k_new, v_new, ref_kc, ref_vc, ids, L if cache else None, gate_cpu)
    gk = kc.to(dev) if kc is not None else None
    gv = vc.to(dev) if vc is not None else None
    g_gate = None
    if qg is not None:
        qg_dev = qg.to(dev)
        g_gate = qg_dev[:, :, D:] if gate == "strided" else qg_dev[:, :, D:].contiguous()
    out = A.paged_attention(q.to(dev), k_new.to(dev), v_new.to(dev), gk, gv, ids, L if cache else None, g_gate)
    torch.cuda.synchronize()
    if cache:
        assert torch.equal(gk.cpu(), ref_kc), "k_cache differs from the oracle's after the call"
        assert torch.equal(gv.cpu(), ref_vc), "v_cache differs from the oracle's after the call"
    return out.cpu(), ref


def _check(out, ref, what):
    assert out.shape == ref.shape, what
    o, r = out.float(), ref.float()
    same = (out.view(torch.int16) == ref.view(torch.int16)).float().mean().item()
    err = (o - r).abs().max().item()
    bound = 1e-2 * r.abs().max().item()
    assert err <= bound, f"{what}: max error {err} above {bound} (identical {same:.4f})"
    assert same >= 0.98, f"{what}: only {same:.4f} of the outputs bit-identical (max error {err})"


# (S, H, Hkv, D, L, block_size, gate): decode at the Qwen3-1.7B / 8B head
# layouts and around the 256-position chunks, MTP verify rows, more rows
# than one launch holds, other head sizes and GQA ratios.
CASES = [
    (1, 16, 8, 128, 1, 16, "none"), (1, 16, 8, 128, 2, 16, "strided"), (1, 16, 8, 128, 255, 16, "none"),
    (1, 16, 8, 128, 256, 16, "contiguous"), (1, 16, 8, 128, 257, 16, "strided"),
    (1, 16, 8, 128, 384, 16, "strided"), (1, 32, 8, 128, 1000, 16, "strided"),
    (1, 32, 8, 128, 4097, 64, "none"), (4, 16, 8, 128, 517, 16, "strided"), (5, 32, 8, 128, 600, 16, "strided"),
    (20, 16, 8, 128, 300, 16, "strided"), (9, 32, 8, 128, 40, 16, "none"), (3, 8, 1, 128, 77, 8, "contiguous"),
    (2, 4, 4, 64, 129, 1, "strided"), (3, 8, 2, 256, 270, 32, "strided"), (1, 64, 2, 128, 33, 16, "none"),
    (4, 16, 8, 128, 512, 16, "strided"), (4, 16, 8, 128, 513, 16, "strided"), (2, 16, 4, 256, 300, 16, "strided"),
    (1, 8, 8, 64, 500, 4, "contiguous"), (1, 8, 2, 256, 300, 16, "strided"), (16, 16, 16, 64, 200, 16, "strided"),
    (4, 16, 8, 128, 700, 16, "strided"), (1, 32, 8, 128, 1025, 16, "none"),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "S{}_H{}_kv{}_D{}_L{}_bs{}_{}".format(*c))
def test_paged_attention_against_oracle(case, dev):
    S, H, Hkv, D, L, BS, gate = case
    _say(f"[gpu] attention {case}")
    out, ref = _run_both(dev, S, H, Hkv, D, L, BS, True, gate, seed=S * 100003 + L)
    _check(out, ref, str(case))


@pytest.mark.parametrize("case", [c for c in CASES if c[4] <= 512], ids=lambda c: "S{}_H{}_kv{}_D{}_L{}".format(*c))
def test_short_context_two_launch_path(case, dev, monkeypatch):
    """Up to 512 positions and 8 rows per kv head run as one launch; the
    two-launch path (scores, then P.V) must give the same results there."""
    monkeypatch.setenv("PILM_HIP_ATTN_SMALL", "0")
    S, H, Hkv, D, L, BS, gate = case
    _say(f"[gpu] attention two-launch {case}")
    out, ref = _run_both(dev, S, H, Hkv, D, L, BS, True, gate, seed=S * 100003 + L)
    _check(out, ref, str(case))


@pytest.mark.parametrize("case", [c for c in CASES if c[0] * (c[1] // c[2]) > 8],
                         ids=lambda c: "S{}_H{}_kv{}_D{}_L{}".format(*c))
def test_without_row_groups(case, dev, monkeypatch):
    """More than 8 query rows per kv head run as row groups of 8 on small
    grids; the single-group kernels (16, 24 or 32 rows) give the same results."""
    monkeypatch.setenv("PILM_HIP_ATTN_ROWGROUPS", "0")
    S, H, Hkv, D, L, BS, gate = case
    _say(f"[gpu] attention one row group {case}")
    out, ref = _run_both(dev, S, H, Hkv, D, L, BS, True, gate, seed=S * 100003 + L)
    _check(out, ref, str(case))


@pytest.mark.parametrize("S,H,Hkv,D", [(1, 16, 8, 128), (33, 16, 8, 128), (7, 32, 8, 64)])
def test_no_cache_prefill(S, H, Hkv, D, dev):
    """attention.py:115-116: the rows attend to each other only (causal)."""
    _say(f"[gpu] attention no cache S={S} H={H} kv={Hkv} D={D}")
    out, ref = _run_both(dev, S, H, Hkv, D, S, cache=False, gate="strided", seed=S)
    _check(out, ref, f"no cache S={S}")


def test_long_context_8b_heads(dev):
    """32768 positions (128 chunks per kv head, the ticket fold over all of
    them) at the Qwen3-8B head layout."""
    _say("[gpu] attention L=32768")
    out, ref = _run_both(dev, 1, 32, 8, 128, 32768, 16, True, "strided", seed=11)
    _check(out, ref, "L=32768")


def test_repeat_calls_identical(dev):
    """Tickets are reset by the last workgroup: the same call twice gives the same bits."""
    q, k_new, v_new, kc, vc, ids, qg = _inputs(3, 4, 16, 8, 128, 1500, 16, True, "strided")
    args = [t.to(dev) for t in (q, k_new, v_new, kc, vc)]
    gate = qg.to(dev)[:, :, 128:]
    o1 = A.paged_attention(*args, ids, 1500, gate)
    o2 = A.paged_attention(*args, ids, 1500, gate)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


def test_paged_kv_cache_class(dev):
    """PagedKVCache.write / read_seq / attend against the oracle's cache."""
    S, H, Hkv, D, L, BS = 2, 16, 8, 128, 50, 16
    q, k_new, v_new, kc, vc, ids, _ = _inputs(5, S, H, Hkv, D, L, BS)
    cache = A.PagedKVCache(1, kc.shape[0], BS, Hkv, D, device=dev)
    cache.k_cache[0].copy_(kc.to(dev))
    cache.v_cache[0].copy_(vc.to(dev))
    out = cache.attend(0, ids, L, q.to(dev), k_new.to(dev), v_new.to(dev))
    ref = OA.paged_attention(q, k_new, v_new, kc, vc, ids, L)
    _check(out.cpu(), ref, "PagedKVCache.attend")
    k, v = cache.read_seq(0, ids[: (L + BS - 1) // BS], L)
    rk, rv = OA.read_seq(kc, vc, ids[: (L + BS - 1) // BS], L)
    assert torch.equal(k.cpu(), rk) and torch.equal(v.cpu(), rv)
    cache.write(0, [ids[0]], [3], k_new[:1].to(dev), v_new[:1].to(dev))
    assert torch.equal(cache.k_cache[0][ids[0], 3].cpu(), k_new[0])


def test_rejected_arguments(dev):
    q, k_new, v_new, kc, vc, ids, _ = _inputs(1, 2, 16, 8, 128, 40, 16)
    gq, gk, gv, gkc, gvc = (t.to(dev) for t in (q, k_new, v_new, kc, vc))
    with pytest.raises(ValueError):
        A.paged_attention(q, k_new, v_new)                      # host tensors
    with pytest.raises(RuntimeError):
        A.paged_attention(gq, gk, gv, gkc, gvc, ids, 1)         # cache_len < S
    with pytest.raises(IndexError):
        A.paged_attention(gq, gk, gv, gkc, gvc, ids[:1], 40)    # too few block ids (a host list, as the reference indexes)
    with pytest.raises(RuntimeError):
        A.paged_attention(gq, gk, gv, gkc, gvc, torch.tensor(ids[:1], dtype=torch.int32, device=dev), 40)   # device table
    with pytest.raises(RuntimeError):
        A.paged_attention(gq, gk, gv, None, None, None, 40)     # no cache needs cache_len == S


@pytest.mark.parametrize("L", [300, 1000, 5000])
def test_graph_replays_match_eager(L, dev):
    """The call captured in a HIP graph (one launch at 300 positions; two
    launches with the P.V ticket at 1000; with the statistics ticket too at
    5000) and replayed three times with eager work in between: every replay
    gives the eager call's bits (tickets are reset by the kernels, no memset
    is captured)."""
    _say(f"[gpu] attention graph L={L}")
    S, H, Hkv, D, BS = 1, 16, 8, 128, 16
    q, k_new, v_new, kc, vc, ids, qg = _inputs(21, S, H, Hkv, D, L, BS, True, "strided")
    args = [t.to(dev) for t in (q, k_new, v_new, kc, vc)]
    table = torch.tensor(ids, dtype=torch.int32, device=dev)
    gate = qg.to(dev)[:, :, D:]
    eager = A.paged_attention(*args, table, L, gate)        # also sizes the scratch before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        A.paged_attention(*args, table, L, gate)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        out = A.paged_attention(*args, table, L, gate)
    # eager work between replays, on caches of its own (a call stores its new
    # rows, which would change what the captured call reads)
    other = [args[0], args[1], args[2], args[3].clone(), args[4].clone()]
    for i in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        junk = A.paged_attention(*other, table, L // 2 + 1, gate)
        torch.cuda.synchronize()
        del junk
