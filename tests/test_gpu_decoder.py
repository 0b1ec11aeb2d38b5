"""GPU: the decoder-step kernels and the device decoder, bit for bit.

Each entry point (ekernel_rmsnorm_gemma_bf16, ekernel_qk_norm_rope_bf16,
ekernel_attention_exact_bf16, ekernel_silu_mul_bf16, ekernel_greedy_step_bf16)
is compared byte for byte with the oracle (oracle/decoder.c, pinned against
torch's CPU kernels and the reference's fixture by test_oracle_decoder.py) on
seeded inputs, through the C ABI.  Then the whole device decoder
(pilm_amd.qwen3) must reproduce the fixtures piLM's own Engine.generate wrote:
the quantized weights' hashes, every step's bf16 logits and the greedy tokens
-- for a two-layer model and for Qwen3-1.7B (128-token prompt, 256 tokens).
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

from oracle import decoder as OD

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _dev16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint16).view(np.int16)).view(torch.bfloat16).to(dev)


def _bits(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _rand16(rng, shape, scale=1.0):
    from pilm_amd import synth as S
    return S.f32_to_bf16_bits((rng.standard_normal(shape) * scale).astype(np.float32)).reshape(shape)


@pytest.fixture(scope="module")
def lib():
    from pilm_amd import bindings as abi
    return abi._load_lib()


def _bind():
    from pilm_amd import bindings as abi
    abi.set_stream(torch.cuda.current_stream().cuda_stream)


def _vp(t):
    import ctypes
    return ctypes.c_void_p(t.data_ptr() if t is not None else None)


# --------------------------------------------------------------- rmsnorm

@pytest.mark.parametrize("rows,n", [(1, 2048), (16, 2048), (3, 4096), (2, 128), (5, 296), (1, 8192), (2, 6144),
                                    (2, 100)])
@pytest.mark.parametrize("with_res", [False, True])
def test_rmsnorm_kernel(lib, dev, rows, n, with_res):
    import ctypes
    from pilm_amd import bindings as abi
    rng = np.random.default_rng(rows * n + with_res)
    x, r, w = _rand16(rng, (rows, n), 3.0), _rand16(rng, (rows, n)), _rand16(rng, (n,), 0.02)
    want, want_res = OD.rmsnorm_gemma_bf16(x, r if with_res else None, w, 1e-6)
    xd, rd, wd = _dev16(x, dev), _dev16(r, dev), _dev16(w, dev)
    out, res_out = torch.empty_like(xd), torch.empty_like(xd)
    _say(f"[gpu] rmsnorm rows={rows} n={n} residual={with_res}")
    _bind()
    d = abi.EkernelRmsnormDesc(rows, n, 1e-6)
    rc = lib.ekernel_rmsnorm_gemma_bf16(ctypes.byref(d), _vp(xd), _vp(rd if with_res else None), _vp(wd), _vp(out),
                                        _vp(res_out if with_res else None))
    assert rc == 0, abi.last_error()
    assert np.array_equal(_bits(out), want)
    if with_res:
        assert np.array_equal(_bits(res_out), want_res)


def test_rmsnorm_in_place_residual(lib, dev):
    """The decoder passes residual and residual_out as one buffer."""
    import ctypes
    from pilm_amd import bindings as abi
    rng = np.random.default_rng(7)
    x, r, w = _rand16(rng, (4, 2048)), _rand16(rng, (4, 2048)), _rand16(rng, (2048,), 0.02)
    want, want_res = OD.rmsnorm_gemma_bf16(x, r, w, 1e-6)
    xd, rd, wd = _dev16(x, dev), _dev16(r, dev), _dev16(w, dev)
    out = torch.empty_like(xd)
    _bind()
    rc = lib.ekernel_rmsnorm_gemma_bf16(ctypes.byref(abi.EkernelRmsnormDesc(4, 2048, 1e-6)), _vp(xd), _vp(rd),
                                        _vp(wd), _vp(out), _vp(rd))
    assert rc == 0
    assert np.array_equal(_bits(out), want) and np.array_equal(_bits(rd), want_res)


def test_rmsnorm_unaligned_rows(lib, dev):
    """Rows that are not 16-byte aligned take the element-wise kernel."""
    import ctypes
    from pilm_amd import bindings as abi
    rng = np.random.default_rng(9)
    x, r, w = _rand16(rng, (3, 2048)), _rand16(rng, (3, 2048)), _rand16(rng, (2048,), 0.02)
    want, want_res = OD.rmsnorm_gemma_bf16(x, r, w, 1e-6)
    xd = torch.empty(3 * 2048 + 1, dtype=torch.bfloat16, device=dev)
    xd[1:].copy_(_dev16(x, dev).reshape(-1))
    rd, wd = _dev16(r, dev), _dev16(w, dev)
    out, res_out = torch.empty((3, 2048), dtype=torch.bfloat16, device=dev), torch.empty_like(rd)
    _bind()
    rc = lib.ekernel_rmsnorm_gemma_bf16(ctypes.byref(abi.EkernelRmsnormDesc(3, 2048, 1e-6)), _vp(xd[1:]), _vp(rd),
                                        _vp(wd), _vp(out), _vp(res_out))
    assert rc == 0, abi.last_error()
    assert np.array_equal(_bits(out), want) and np.array_equal(_bits(res_out), want_res)


# ----------------------------------------------------- norm + W4A16 g128 linear

@pytest.mark.parametrize("N,K,swiglu,with_res", [(6144, 2048, False, True), (12288, 2048, True, True),
                                                 (1536, 256, False, False), (1024, 256, True, True),
                                                 (10240, 4096, False, True), (24576, 4096, True, True),
                                                 (2048, 2048, False, False), (48, 512, True, False),
                                                 (512, 12288, False, True)])
def test_rmsnorm_linear_fused(lib, dev, N, K, swiglu, with_res):
    """ekernel_rmsnorm_linear_w4a16g128_bf16 against the oracle's GemmaRMSNorm,
    W4A16 g128 linear and (swiglu) F.silu(gate) * up, bit for bit: Qwen3-1.7B
    and 8B q/k/v and gate/up shapes, the two-layer model's, and small ones."""
    import ctypes
    from oracle import oracle as O
    from pilm_amd import bindings as abi
    rng = np.random.default_rng(N + K + swiglu)
    x, r, nw = _rand16(rng, (1, K), 3.0), _rand16(rng, (1, K)), _rand16(rng, (K,), 0.02)
    q = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    sc = (rng.random((N, K // 128)) * 0.019 + 0.001).astype(np.float32)
    a, h = OD.rmsnorm_gemma_bf16(x, r if with_res else None, nw, 1e-6)
    y = O.linear_w4a16g_bf16(a, q, sc, 128)
    if swiglu:
        half = N // 2
        want = OD.silu_mul_bf16(np.ascontiguousarray(y[:, :half]), np.ascontiguousarray(y[:, half:]), 1, half, half)
    else:
        want = y
    xd, rd, nwd = _dev16(x, dev), _dev16(r, dev), _dev16(nw, dev)
    qd, sd = torch.from_numpy(q).to(dev), torch.from_numpy(sc).to(dev)
    out = torch.empty((1, N // 2 if swiglu else N), dtype=torch.bfloat16, device=dev)
    res_out = torch.empty((1, K), dtype=torch.bfloat16, device=dev)
    _say(f"[gpu] rmsnorm + linear N={N} K={K} swiglu={swiglu} residual={with_res}")
    _bind()
    d = abi.EkernelNormLinearDesc(1, N, K, 1e-6, int(swiglu))
    rc = lib.ekernel_rmsnorm_linear_w4a16g128_bf16(ctypes.byref(d), _vp(xd), _vp(rd if with_res else None), _vp(nwd),
                                                   _vp(res_out if with_res else None), _vp(qd), _vp(sd), _vp(out))
    assert rc == 0, abi.last_error()
    got = _bits(out)
    bad = np.argwhere(got != want.reshape(got.shape))
    assert len(bad) == 0, f"{len(bad)} outputs differ, first {bad[:4].tolist()}"
    if with_res:
        assert np.array_equal(_bits(res_out), h)


def test_rmsnorm_linear_fused_refuses(lib, dev):
    """Two rows, K not a multiple of 256, misaligned rows and outputs that
    overlap the inputs are refused before any launch."""
    import ctypes
    from pilm_amd import bindings as abi
    buf = torch.zeros(1 << 20, dtype=torch.bfloat16, device=dev)
    q = torch.zeros((64, 1024), dtype=torch.uint8, device=dev)
    sc = torch.ones((64, 16), dtype=torch.float32, device=dev)
    _bind()
    p = buf.data_ptr()

    def call(rows, N, K, x, res, res_out, out, swiglu=0):
        d = abi.EkernelNormLinearDesc(rows, N, K, 1e-6, swiglu)
        return lib.ekernel_rmsnorm_linear_w4a16g128_bf16(ctypes.byref(d), ctypes.c_void_p(x),
                                                         ctypes.c_void_p(res) if res else None,
                                                         ctypes.c_void_p(p + 65536),
                                                         ctypes.c_void_p(res_out) if res_out else None, _vp(q),
                                                         _vp(sc), ctypes.c_void_p(out))
    assert call(1, 64, 2048, p, p + 8192, p + 16384, p + 32768) == 0
    assert call(2, 64, 2048, p, p + 8192, p + 16384, p + 32768) == abi.ECPU_ERR_UNSUPPORTED
    assert call(1, 64, 2000, p, p + 8192, p + 16384, p + 32768) == abi.ECPU_ERR_UNSUPPORTED
    assert call(1, 64, 2048, p + 2, p + 8192, p + 16384, p + 32768) == abi.ECPU_ERR_UNSUPPORTED
    assert call(1, 64, 2048, p, p + 8192, p + 8192, p + 32768) == abi.ECPU_ERR_PARAM       # residual_out = residual
    assert call(1, 64, 2048, p, p + 8192, p + 16384, p + 1024) == abi.ECPU_ERR_PARAM       # out inside x
    assert call(1, 24, 2048, p, p + 8192, p + 16384, p + 32768, swiglu=1) == abi.ECPU_ERR_UNSUPPORTED
    torch.cuda.synchronize()


# ----------------------------------------------------- q/k norm + rope + attention

def _attn_case(rng, S, H, Hkv, D, pos0, bs=16, spare=3):
    L = pos0 + S
    nblk = (L + bs - 1) // bs
    nphys = nblk + spare
    block_ids = rng.permutation(nphys)[:nblk].astype(np.int32)
    kc = _rand16(rng, (nphys, bs, Hkv, D))
    vc = _rand16(rng, (nphys, bs, Hkv, D))
    qkv = _rand16(rng, (S, (2 * H + 2 * Hkv) * D))          # fused [q | gate per head][k][v]
    qw, kw = _rand16(rng, (D,), 0.02), _rand16(rng, (D,), 0.02)
    return L, block_ids, kc, vc, qkv, qw, kw


@pytest.mark.parametrize("S,H,Hkv,D,pos0", [(1, 16, 8, 128, 383), (16, 16, 8, 128, 112), (16, 16, 8, 128, 0),
                                            (5, 32, 8, 128, 2043), (1, 4, 2, 128, 0), (3, 8, 8, 64, 17),
                                            (2, 4, 1, 256, 40), (1, 16, 8, 128, 2), (1, 16, 8, 128, 7)])
def test_qk_rope_then_attention(lib, dev, S, H, Hkv, D, pos0):
    import ctypes
    from pilm_amd import bindings as abi
    rng = np.random.default_rng(S * 7919 + pos0 + H)
    bs = 16
    L, block_ids, kc, vc, qkv, qw, kw = _attn_case(rng, S, H, Hkv, D, pos0, bs)
    cos, sin = OD.rope_tables(1e6, D, L + 1)
    stride = qkv.shape[1]
    qg, k, v = qkv[:, :2 * H * D], qkv[:, 2 * H * D:2 * H * D + Hkv * D], qkv[:, 2 * H * D + Hkv * D:]
    kc_o, vc_o = kc.copy(), vc.copy()
    q_want = OD.qk_norm_rope_bf16(qg, k, v, qw, kw, cos, sin, pos0, kc_o, vc_o, block_ids, n_heads=H, n_kv_heads=Hkv,
                                  head_dim=D, rot_dim=D, eps=1e-6, block_size=bs)
    gate = qkv.reshape(-1)[D:]
    want = OD.attention_exact_bf16(q_want, kc_o, vc_o, block_ids, L, gate, stride, 2 * D, block_size=bs)

    qkv_d, kc_d, vc_d = _dev16(qkv, dev), _dev16(kc, dev), _dev16(vc, dev)
    bid_d = torch.from_numpy(block_ids).to(dev)
    cos_d, sin_d = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    qw_d, kw_d = _dev16(qw, dev), _dev16(kw, dev)
    q_d = torch.empty((S, H, D), dtype=torch.bfloat16, device=dev)
    out_d = torch.empty((S, H * D), dtype=torch.bfloat16, device=dev)
    step = torch.tensor([pos0, L, 0, 0], dtype=torch.int32, device=dev)
    nblk = len(block_ids)
    _say(f"[gpu] qk rope + attention S={S} H={H} Hkv={Hkv} D={D} pos0={pos0}")
    _bind()
    p = qkv_d.data_ptr()
    for use_step in (False, True):
        kc_d.copy_(_dev16(kc, dev))
        vc_d.copy_(_dev16(vc, dev))
        rd = abi.EkernelQkRopeDesc(S, H, Hkv, D, D, stride, stride, pos0, L + 1, bs, kc.shape[0], nblk, 1e-6)
        rc = lib.ekernel_qk_norm_rope_bf16(ctypes.byref(rd), ctypes.c_void_p(p), ctypes.c_void_p(p + 2 * H * D * 2),
                                           ctypes.c_void_p(p + (2 * H * D + Hkv * D) * 2), _vp(qw_d), _vp(kw_d),
                                           _vp(cos_d), _vp(sin_d), _vp(step if use_step else None), _vp(q_d),
                                           _vp(kc_d), _vp(vc_d), _vp(bid_d))
        assert rc == 0, abi.last_error()
        assert np.array_equal(_bits(q_d), q_want)
        assert np.array_equal(_bits(kc_d), kc_o) and np.array_equal(_bits(vc_d), vc_o)
        ad = abi.EkernelAttentionExactDesc(S, H, Hkv, D, L, bs, kc.shape[0], nblk, stride, 2 * D)
        rc = lib.ekernel_attention_exact_bf16(ctypes.byref(ad), _vp(q_d), _vp(kc_d), _vp(vc_d), _vp(bid_d),
                                              ctypes.c_void_p(p + D * 2), _vp(step if use_step else None), _vp(out_d))
        assert rc == 0, abi.last_error()
        got = _bits(out_d)
        bad = np.argwhere(got != want)
        assert len(bad) == 0, f"{len(bad)} outputs differ, first {bad[:4].tolist()} (step={use_step})"


@pytest.mark.parametrize("H,Hkv,D,plan", [
    (16, 8, 128, [(5, 130), (5, 0), (1, 47), (5, 16), (3, 2), (5, 255), (1, 0), (4, 60)]),
    (32, 8, 128, [(5, 300), (5, 31), (5, 0), (5, 511)]),
    (8, 8, 64, [(2, 3), (7, 40), (1, 1)]),
    (16, 8, 128, [(5, p) for p in range(0, 256, 16)]),                   # 16 sequences x 5 rows: M = 80
    (16, 8, 128, [(16, 0), (16, 16), (13, 100), (9, 200), (16, 480), (2, 5)]),   # prefill chunks, long rows
    (8, 8, 64, [(16, 48), (11, 3), (16, 0), (1, 700)]),
])
def test_rope_attention_batch_matches_per_sequence(lib, dev, monkeypatch, H, Hkv, D, plan):
    """ekernel_qk_norm_rope_batch_bf16 + ekernel_attention_exact_batch_bf16:
    several sequences (rows, pos0) with their own block tables in one shared
    pool, listed out of table order, in one call each; every q row, cache row
    and output row equal to the oracle's per-sequence steps.  The attention
    runs with every tiling: the per-row kernel (PILM_HIP_ATTN_TILE=0), the
    chosen tile rows, one row per tile, three (ragged tiles) and the most a
    tile holds (16 (row, q head) vectors)."""
    import ctypes
    from pilm_amd import bindings as abi
    rng = np.random.default_rng(len(plan) * 131 + H + D)
    bs, nseq = 16, len(plan)
    per = max((p + n + bs - 1) // bs for n, p in plan) + 1         # blocks per table
    nphys = nseq * per + 5
    perm = rng.permutation(nphys).astype(np.int32)
    tables = perm[:nseq * per].reshape(nseq, per)                  # disjoint physical blocks per sequence
    kc = _rand16(rng, (nphys, bs, Hkv, D))
    vc = _rand16(rng, (nphys, bs, Hkv, D))
    rows = sum(n for n, _ in plan)
    width = (2 * H + 2 * Hkv) * D
    qkv = _rand16(rng, (rows, width))
    qw, kw = _rand16(rng, (D,), 0.02), _rand16(rng, (D,), 0.02)
    max_pos = per * bs
    cos, sin = OD.rope_tables(1e6, D, max_pos)
    order = rng.permutation(nseq)          # batch rows follow this order; sequence i keeps table i
    row0, r = {}, 0
    for i in order:
        row0[i] = r
        r += plan[i][0]
    kc_o, vc_o = kc.copy(), vc.copy()
    q_want = np.zeros((rows, H, D), dtype=np.uint16)
    out_want = np.zeros((rows, H * D), dtype=np.uint16)
    for i in range(nseq):
        n, p0 = plan[i]
        blk = qkv[row0[i]:row0[i] + n]
        qg, k, v = blk[:, :2 * H * D], blk[:, 2 * H * D:2 * H * D + Hkv * D], blk[:, 2 * H * D + Hkv * D:]
        qi = OD.qk_norm_rope_bf16(qg, k, v, qw, kw, cos, sin, p0, kc_o, vc_o, tables[i], n_heads=H, n_kv_heads=Hkv,
                                  head_dim=D, rot_dim=D, eps=1e-6, block_size=bs)
        q_want[row0[i]:row0[i] + n] = qi.reshape(n, H, D)
        gate = blk.reshape(-1)[D:]
        out_want[row0[i]:row0[i] + n] = OD.attention_exact_bf16(qi, kc_o, vc_o, tables[i], p0 + n, gate, width,
                                                                2 * D, block_size=bs).reshape(n, H * D)
    qkv_d, kc_d, vc_d = _dev16(qkv, dev), _dev16(kc, dev), _dev16(vc, dev)
    tab_d = torch.from_numpy(tables.reshape(-1).copy()).to(dev)
    cos_d, sin_d = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    qw_d, kw_d = _dev16(qw, dev), _dev16(kw, dev)
    q_d = torch.empty((rows, H, D), dtype=torch.bfloat16, device=dev)
    out_d = torch.empty((rows, H * D), dtype=torch.bfloat16, device=dev)
    seqs = (abi.EkernelBatchSeq * nseq)(*[abi.EkernelBatchSeq(row0[i], plan[i][0], plan[i][1], i) for i in order])
    _say(f"[gpu] batched rope + attention H={H} Hkv={Hkv} D={D} {nseq} sequences, {rows} rows")
    _bind()
    p = qkv_d.data_ptr()
    rd = abi.EkernelQkRopeDesc(rows, H, Hkv, D, D, width, width, 0, max_pos, bs, nphys, per, 1e-6)
    rc = lib.ekernel_qk_norm_rope_batch_bf16(ctypes.byref(rd), seqs, nseq, nseq, ctypes.c_void_p(p),
                                             ctypes.c_void_p(p + 2 * H * D * 2),
                                             ctypes.c_void_p(p + (2 * H * D + Hkv * D) * 2), _vp(qw_d), _vp(kw_d),
                                             _vp(cos_d), _vp(sin_d), _vp(q_d), _vp(kc_d), _vp(vc_d), _vp(tab_d))
    assert rc == 0, abi.last_error()
    assert np.array_equal(_bits(q_d), q_want)
    assert np.array_equal(_bits(kc_d), kc_o) and np.array_equal(_bits(vc_d), vc_o)
    ad = abi.EkernelAttentionExactDesc(rows, H, Hkv, D, 0, bs, nphys, per, width, 2 * D)
    for tile, tile_rows in (("0", "0"), ("1", "0"), ("1", "1"), ("1", "3"), ("1", "16")):
        monkeypatch.setenv("PILM_HIP_ATTN_TILE", tile)
        monkeypatch.setenv("PILM_HIP_ATTN_TILE_ROWS", tile_rows)
        _say(f"[gpu]   attention, tile kernel {tile}, rows per tile {tile_rows}")
        out_d.fill_(0)
        rc = lib.ekernel_attention_exact_batch_bf16(ctypes.byref(ad), seqs, nseq, nseq, _vp(q_d), _vp(kc_d),
                                                    _vp(vc_d), _vp(tab_d), ctypes.c_void_p(p + D * 2), _vp(out_d))
        assert rc == 0, abi.last_error()
        got = _bits(out_d)
        bad = np.argwhere(got != out_want)
        assert len(bad) == 0, f"{len(bad)} outputs differ (tile {tile}/{tile_rows}), first {bad[:4].tolist()}"


def test_attention_batch_long_sequence(lib, dev):
    """A sequence of 8002 positions beside a short one in one batched
    attention call (the scores of a row no longer fit 64 KB: the tile kernel
    takes the workgroup's whole LDS); outputs equal to the oracle's."""
    import ctypes
    from pilm_amd import bindings as abi
    rng = np.random.default_rng(8000)
    H, Hkv, D, bs = 16, 8, 128, 16
    plan = [(2, 8000), (5, 100)]
    per = max((p + n + bs - 1) // bs for n, p in plan)
    nseq = len(plan)
    nphys = nseq * per
    tables = rng.permutation(nphys).astype(np.int32).reshape(nseq, per)
    kc, vc = _rand16(rng, (nphys, bs, Hkv, D)), _rand16(rng, (nphys, bs, Hkv, D))
    rows = sum(n for n, _ in plan)
    width = (2 * H + 2 * Hkv) * D
    qkv = _rand16(rng, (rows, width))
    q = _rand16(rng, (rows, H, D))
    want = np.zeros((rows, H * D), np.uint16)
    r0 = 0
    for i, (n, p0) in enumerate(plan):
        want[r0:r0 + n] = OD.attention_exact_bf16(q[r0:r0 + n], kc, vc, tables[i], p0 + n,
                                                  qkv[r0:r0 + n].reshape(-1)[D:], width, 2 * D,
                                                  block_size=bs).reshape(n, H * D)
        r0 += n
    q_d, kc_d, vc_d, qkv_d = _dev16(q, dev), _dev16(kc, dev), _dev16(vc, dev), _dev16(qkv, dev)
    tab_d = torch.from_numpy(tables.reshape(-1).copy()).to(dev)
    out_d = torch.zeros((rows, H * D), dtype=torch.bfloat16, device=dev)
    seqs = (abi.EkernelBatchSeq * nseq)(abi.EkernelBatchSeq(0, 2, 8000, 0), abi.EkernelBatchSeq(2, 5, 100, 1))
    _say("[gpu] batched attention, 8002 and 105 positions")
    _bind()
    ad = abi.EkernelAttentionExactDesc(rows, H, Hkv, D, 0, bs, nphys, per, width, 2 * D)
    rc = lib.ekernel_attention_exact_batch_bf16(ctypes.byref(ad), seqs, nseq, nseq, _vp(q_d), _vp(kc_d), _vp(vc_d),
                                                _vp(tab_d), ctypes.c_void_p(qkv_d.data_ptr() + D * 2), _vp(out_d))
    assert rc == 0, abi.last_error()
    assert np.array_equal(_bits(out_d), want)


def test_rope_attention_batch_rejects_bad_tables(lib, dev):
    """Rows in two sequences or in none, a table index beyond n_tables,
    positions beyond the tables and more than 128 rows are refused before
    anything is launched."""
    import ctypes
    from pilm_amd import bindings as abi
    H, Hkv, D, bs, per, nphys = 4, 2, 64, 16, 4, 16
    buf = torch.zeros(1 << 20, dtype=torch.bfloat16, device=dev)
    tab = torch.arange(8, dtype=torch.int32, device=dev)
    p = buf.data_ptr()

    def att(rows, plan, n_tables=2):
        seqs = (abi.EkernelBatchSeq * len(plan))(*[abi.EkernelBatchSeq(*x) for x in plan])
        ad = abi.EkernelAttentionExactDesc(rows, H, Hkv, D, 0, bs, nphys, per, 0, 0)
        return lib.ekernel_attention_exact_batch_bf16(ctypes.byref(ad), seqs, len(plan), n_tables,
                                                      ctypes.c_void_p(p), ctypes.c_void_p(p + 65536),
                                                      ctypes.c_void_p(p + 131072), _vp(tab), None,
                                                      ctypes.c_void_p(p + 262144))
    _bind()
    assert att(4, [(0, 2, 0, 0), (2, 2, 5, 1)]) == 0
    assert att(4, [(0, 3, 0, 0), (2, 2, 5, 1)]) == abi.ECPU_ERR_PARAM          # row 2 in two sequences
    assert att(5, [(0, 2, 0, 0), (2, 2, 5, 1)]) == abi.ECPU_ERR_PARAM          # row 4 in none
    assert att(4, [(0, 2, 0, 0), (2, 2, 5, 2)]) == abi.ECPU_ERR_PARAM          # table 2 of 2
    assert att(4, [(0, 2, 0, 0), (2, 2, 63, 1)]) == abi.ECPU_ERR_PARAM         # positions 63, 64 of 64
    assert att(130, [(0, 130, 0, 0)], 1) == abi.ECPU_ERR_UNSUPPORTED           # more than 128 rows
    torch.cuda.synchronize()


@pytest.mark.parametrize("H,Hkv,D,pos0", [(16, 8, 128, 383), (16, 8, 128, 0), (16, 8, 128, 1), (16, 8, 128, 2),
                                          (16, 8, 128, 3), (16, 8, 128, 7), (16, 8, 128, 64), (32, 8, 128, 2043),
                                          (4, 2, 128, 0), (8, 8, 64, 17), (16, 4, 128, 100), (16, 8, 128, 4000),
                                          (32, 8, 64, 515), (16, 8, 128, 511), (16, 8, 128, 512),
                                          (16, 8, 64, 255), (8, 2, 64, 300)])
@pytest.mark.parametrize("shared", [False, True])
def test_decode_attention_fused(lib, dev, H, Hkv, D, pos0, shared, monkeypatch):
    """ekernel_decode_attention_bf16 (one launch) against the oracle's two
    steps: the same output bits and the same cache rows, with the position
    from the host and from the device state word.  Cases: lengths 1-4
    (torch's small-matrix kernel below 4), 8 and 65 (tails of the four- and
    eight-way sums), 1, 2 and 4 q heads per kv head, value rows staged in one
    pass and in several (2044 and 4001 positions); one q head per workgroup
    and (shared) all q heads of a kv head per workgroup.  With one q head per
    workgroup, 512 positions are the last that take the value rows through
    registers and the workgroup-wide softmax, 513 the first staged by copy
    after the scores."""
    import ctypes
    from pilm_amd import bindings as abi
    monkeypatch.setenv("PILM_DECODE_ATTN_SHARED", "1" if shared else "0")
    rng = np.random.default_rng(pos0 * 31 + H + D)
    bs, S = 16, 1
    L, block_ids, kc, vc, qkv, qw, kw = _attn_case(rng, S, H, Hkv, D, pos0, bs)
    cos, sin = OD.rope_tables(1e6, D, L + 1)
    stride = qkv.shape[1]
    qg, k, v = qkv[:, :2 * H * D], qkv[:, 2 * H * D:2 * H * D + Hkv * D], qkv[:, 2 * H * D + Hkv * D:]
    kc_o, vc_o = kc.copy(), vc.copy()
    q_want = OD.qk_norm_rope_bf16(qg, k, v, qw, kw, cos, sin, pos0, kc_o, vc_o, block_ids, n_heads=H, n_kv_heads=Hkv,
                                  head_dim=D, rot_dim=D, eps=1e-6, block_size=bs)
    want = OD.attention_exact_bf16(q_want, kc_o, vc_o, block_ids, L, qkv.reshape(-1)[D:], stride, 2 * D,
                                   block_size=bs)
    qkv_d, kc_d, vc_d = _dev16(qkv, dev), _dev16(kc, dev), _dev16(vc, dev)
    bid_d = torch.from_numpy(block_ids).to(dev)
    cos_d, sin_d = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    qw_d, kw_d = _dev16(qw, dev), _dev16(kw, dev)
    out_d = torch.empty((1, H * D), dtype=torch.bfloat16, device=dev)
    step = torch.tensor([pos0, L, 0, 0], dtype=torch.int32, device=dev)
    _say(f"[gpu] fused decode attention H={H} Hkv={Hkv} D={D} pos0={pos0}")
    _bind()
    p = qkv_d.data_ptr()
    for use_step in (False, True):
        kc_d.copy_(_dev16(kc, dev))
        vc_d.copy_(_dev16(vc, dev))
        out_d.zero_()
        rd = abi.EkernelQkRopeDesc(1, H, Hkv, D, D, stride, stride, pos0, L + 1, bs, kc.shape[0], len(block_ids), 1e-6)
        rc = lib.ekernel_decode_attention_bf16(ctypes.byref(rd), ctypes.c_void_p(p),
                                               ctypes.c_void_p(p + 2 * H * D * 2),
                                               ctypes.c_void_p(p + (2 * H * D + Hkv * D) * 2), _vp(qw_d), _vp(kw_d),
                                               _vp(cos_d), _vp(sin_d), _vp(step if use_step else None), _vp(kc_d),
                                               _vp(vc_d), _vp(bid_d), _vp(out_d))
        assert rc == 0, abi.last_error()
        assert np.array_equal(_bits(kc_d), kc_o) and np.array_equal(_bits(vc_d), vc_o)
        got = _bits(out_d)
        bad = np.argwhere(got != want)
        assert len(bad) == 0, f"{len(bad)} outputs differ, first {bad[:4].tolist()} (step={use_step})"


@pytest.mark.parametrize("pos0", [100, 511])
def test_decode_attention_fused_long_table(lib, dev, pos0):
    """A short row in block tables and rope tables sized for 32768 positions
    (the decoder sized for long sequences): accepted, with the oracle's
    output and cache rows, as in a table sized to fit."""
    import ctypes
    from pilm_amd import bindings as abi
    rng = np.random.default_rng(pos0 + 77)
    H, Hkv, D, bs, cap = 16, 8, 128, 16, 32768
    L, block_ids, kc, vc, qkv, qw, kw = _attn_case(rng, 1, H, Hkv, D, pos0, bs)
    ids_long = np.concatenate([block_ids, np.zeros(cap // bs - len(block_ids), np.int32)])
    cos, sin = OD.rope_tables(1e6, D, cap)
    stride = qkv.shape[1]
    qg, k, v = qkv[:, :2 * H * D], qkv[:, 2 * H * D:2 * H * D + Hkv * D], qkv[:, 2 * H * D + Hkv * D:]
    kc_o, vc_o = kc.copy(), vc.copy()
    q_want = OD.qk_norm_rope_bf16(qg, k, v, qw, kw, cos, sin, pos0, kc_o, vc_o, block_ids, n_heads=H, n_kv_heads=Hkv,
                                  head_dim=D, rot_dim=D, eps=1e-6, block_size=bs)
    want = OD.attention_exact_bf16(q_want, kc_o, vc_o, block_ids, L, qkv.reshape(-1)[D:], stride, 2 * D,
                                   block_size=bs)
    qkv_d, kc_d, vc_d = _dev16(qkv, dev), _dev16(kc, dev), _dev16(vc, dev)
    bid_d = torch.from_numpy(ids_long).to(dev)
    cos_d, sin_d = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    qw_d, kw_d = _dev16(qw, dev), _dev16(kw, dev)
    out_d = torch.zeros((1, H * D), dtype=torch.bfloat16, device=dev)
    _say(f"[gpu] fused decode attention, {cap}-position tables, pos0={pos0}")
    _bind()
    p = qkv_d.data_ptr()
    rd = abi.EkernelQkRopeDesc(1, H, Hkv, D, D, stride, stride, pos0, cap, bs, kc.shape[0], len(ids_long), 1e-6)
    rc = lib.ekernel_decode_attention_bf16(ctypes.byref(rd), ctypes.c_void_p(p), ctypes.c_void_p(p + 2 * H * D * 2),
                                           ctypes.c_void_p(p + (2 * H * D + Hkv * D) * 2), _vp(qw_d), _vp(kw_d),
                                           _vp(cos_d), _vp(sin_d), None, _vp(kc_d), _vp(vc_d), _vp(bid_d),
                                           _vp(out_d))
    assert rc == 0, abi.last_error()
    assert np.array_equal(_bits(kc_d), kc_o) and np.array_equal(_bits(vc_d), vc_o)
    assert np.array_equal(_bits(out_d), want)


def test_decode_attention_fused_refuses_unsupported(lib, dev):
    """Other than 1, 2 or 4 q heads per kv head, 256-wide heads and S > 1 are
    refused (the two-call path serves them)."""
    import ctypes
    from pilm_amd import bindings as abi
    buf = torch.zeros(1 << 20, dtype=torch.bfloat16, device=dev)
    cs = torch.zeros(1 << 16, dtype=torch.float32, device=dev)
    bid = torch.zeros(4, dtype=torch.int32, device=dev)
    _bind()
    for S, H, Hkv, D in ((1, 16, 2, 128), (1, 6, 2, 128), (1, 4, 2, 256), (2, 4, 2, 128)):
        rd = abi.EkernelQkRopeDesc(S, H, Hkv, D, D, 0, 0, 0, 16, 16, 4, 4, 1e-6)
        rc = lib.ekernel_decode_attention_bf16(ctypes.byref(rd), _vp(buf), _vp(buf), _vp(buf), _vp(buf), _vp(buf),
                                               _vp(cs), _vp(cs), None, _vp(buf), _vp(buf), _vp(bid), _vp(buf))
        assert rc == abi.ECPU_ERR_UNSUPPORTED, (S, H, Hkv, D, rc)


@pytest.mark.parametrize("L", [1, 2, 3, 4, 5, 8, 9, 64, 65, 129, 512])
def test_attention_decode_lengths_no_gate(lib, dev, L):
    """Decode over every small length (torch's small-matrix kernel below four
    positions, the tail rules of the four- and eight-way sums) and chunk edges,
    without the gate."""
    import ctypes
    from pilm_amd import bindings as abi
    rng = np.random.default_rng(L)
    H, Hkv, D, bs = 16, 8, 128, 16
    nblk = (L + bs - 1) // bs
    block_ids = np.arange(nblk, dtype=np.int32)[::-1].copy()
    kc, vc = _rand16(rng, (nblk, bs, Hkv, D), 2.0), _rand16(rng, (nblk, bs, Hkv, D))
    q = _rand16(rng, (1, H, D), 2.0)
    want = OD.attention_exact_bf16(q, kc, vc, block_ids, L, block_size=bs)
    out = torch.empty((1, H * D), dtype=torch.bfloat16, device=dev)
    _bind()
    _say(f"[gpu] attention decode L={L}")
    ad = abi.EkernelAttentionExactDesc(1, H, Hkv, D, L, bs, nblk, nblk, 0, 0)
    qd, kd, vd = _dev16(q, dev), _dev16(kc, dev), _dev16(vc, dev)     # held: the kernel reads them
    bd = torch.from_numpy(block_ids).to(dev)
    rc = lib.ekernel_attention_exact_bf16(ctypes.byref(ad), _vp(qd), _vp(kd), _vp(vd), _vp(bd), None, None,
                                          _vp(out))
    assert rc == 0, abi.last_error()
    assert np.array_equal(_bits(out), want)


def test_attention_rejects_bad_arguments(lib, dev):
    import ctypes
    from pilm_amd import bindings as abi
    q = torch.zeros((1, 4, 128), dtype=torch.bfloat16, device=dev)
    kc = torch.zeros((2, 16, 2, 128), dtype=torch.bfloat16, device=dev)
    bid = torch.zeros(2, dtype=torch.int32, device=dev)
    out = torch.empty((1, 512), dtype=torch.bfloat16, device=dev)
    _bind()
    for desc in (abi.EkernelAttentionExactDesc(1, 4, 2, 128, 33, 16, 2, 2, 0, 0),    # cache_len > table
                 abi.EkernelAttentionExactDesc(1, 4, 3, 128, 8, 16, 2, 2, 0, 0),     # heads % kv heads
                 abi.EkernelAttentionExactDesc(1, 4, 2, 96, 8, 16, 2, 2, 0, 0)):     # head_dim
        assert lib.ekernel_attention_exact_bf16(ctypes.byref(desc), _vp(q), _vp(kc), _vp(kc), _vp(bid), None, None,
                                                _vp(out)) != 0
    host = torch.zeros((1, 4, 128), dtype=torch.bfloat16)
    desc = abi.EkernelAttentionExactDesc(1, 4, 2, 128, 8, 16, 2, 2, 0, 0)
    assert lib.ekernel_attention_exact_bf16(ctypes.byref(desc), _vp(host), _vp(kc), _vp(kc), _vp(bid), None, None,
                                            _vp(out)) == -1


# ------------------------------------------------------------ silu, greedy

def test_silu_mul_every_bf16_gate(lib, dev):
    rng = np.random.default_rng(3)
    n = 65536
    g = np.arange(n, dtype=np.uint32).astype(np.uint16).reshape(4, n // 4)
    u = _rand16(rng, (4, n // 4))
    gu = np.concatenate([g, u], axis=1)                     # one [rows, 2I] buffer as the decoder has it
    want = OD.silu_mul_bf16(g, u, 4, n // 4, n // 4)
    gd = _dev16(gu, dev)
    out = torch.empty((4, n // 4), dtype=torch.bfloat16, device=dev)
    _bind()
    p = gd.data_ptr()
    import ctypes
    rc = lib.ekernel_silu_mul_bf16(ctypes.c_void_p(p), ctypes.c_void_p(p + (n // 4) * 2), 4, n // 4, n // 2,
                                   _vp(out))
    assert rc == 0
    from pilm_amd import synth as S
    fin = np.isfinite(S.bf16_bits_to_f32(g)) & np.isfinite(S.bf16_bits_to_f32(want))
    assert np.array_equal(_bits(out)[fin], want[fin])


@pytest.mark.parametrize("n", [1, 5, 4096, 151936])
def test_greedy_step(lib, dev, n):
    rng = np.random.default_rng(n)
    logits = _rand16(rng, (n,), 3.0)
    if n > 100:
        top = logits.view(np.uint16)[np.argmax(_f(logits))]
        logits[[n // 3, n - 2]] = top                      # ties: the lowest index wins
    want = OD.argmax_bf16(logits)
    ld = _dev16(logits, dev)
    state = torch.tensor([10, 11, 2, 0], dtype=torch.int32, device=dev)
    toks = torch.full((4,), -1, dtype=torch.int32, device=dev)
    nid = torch.zeros(1, dtype=torch.int64, device=dev)
    _bind()
    assert lib.ekernel_greedy_step_bf16(_vp(ld), n, _vp(state), _vp(toks), 4, _vp(nid)) == 0
    torch.cuda.synchronize()
    assert state.tolist() == [11, 12, 3, 0]
    assert toks.tolist() == [-1, -1, want, -1] and nid.item() == want


def _f(b):
    from pilm_amd import synth as S
    return S.bf16_bits_to_f32(b)


# --------------------------------------------------------- the whole decoder

def _fixture(name):
    return json.loads((GOLDEN / f"decode_{name}.json").read_text())


def _decoder(fx, dev, hashes):
    from pilm_amd import qwen3 as Q
    c = fx["config"]
    cfg = Q.Qwen3Config.from_dict(c)
    w = Q.Qwen3Weights.synthetic(cfg, c["seed"], c["std"], device=dev, hashes=hashes)
    return w, Q.Qwen3Decoder(w, max_positions=c["prompt"] + c["new_tokens"] + 1, max_new_tokens=c["new_tokens"])


def test_decoder_tiny_matches_reference(dev):
    fx = _fixture("tiny")
    _say("[gpu] decoder, two-layer model: weights")
    w, dec = _decoder(fx, dev, hashes=True)
    assert w.quantized_sha == fx["quantized_sha"]
    shas = []
    _say("[gpu] decoder, two-layer model: eager steps with logits")
    toks = dec.generate(fx["prompt"], len(fx["tokens"]), on_logits=lambda i, lg: shas.append(OD.sha_u16(_bits(lg))))
    want = [lg["sha"] for lg in fx["logits"]]
    first = next((i for i, (a, b) in enumerate(zip(shas, want)) if a != b), None)
    assert first is None, f"logits differ first at step {first}"
    assert toks == fx["tokens"]
    _say("[gpu] decoder, two-layer model: graph replay")
    from pilm_amd import qwen3 as Q
    dec2 = Q.Qwen3Decoder(w, max_positions=dec.max_pos, max_new_tokens=dec.max_new)
    assert dec2.generate(fx["prompt"], len(fx["tokens"]), graph=True) == fx["tokens"]
    # a second sequence on the same decoder (graph already captured) starts clean
    assert dec2.generate(fx["prompt"], len(fx["tokens"]), graph=True) == fx["tokens"]
    _say("[gpu] decoder, two-layer model: norm, attention and SwiGLU as separate launches")
    dec3 = Q.Qwen3Decoder(w, max_positions=dec.max_pos, max_new_tokens=dec.max_new)
    dec3.fused_decode = dec3.fused_norm = False
    assert dec3.generate(fx["prompt"], len(fx["tokens"]), graph=True) == fx["tokens"]


def test_decoder_tiny_w8_matches_oracle(dev):
    """The two-layer model with every Linear int8 per output row (the
    reference's W8A32 quantization in a bf16 model runs them as W8A16,
    linear.py:210-231): quantized weights, every step's logits and the greedy
    tokens equal to the oracle's (oracle/decoder.py), eager and replayed.
    The norms run as their own launches (the norm-fused GEMV is W4A16 g128)."""
    from pilm_amd import qwen3 as Q
    c = dict(_fixture("tiny")["config"])
    c["weights"], c["new_tokens"] = "w8", 16
    prompt = _fixture("tiny")["prompt"]
    _say("[gpu] decoder, two-layer W8 model: oracle (CPU)")
    od = OD.OracleDecoder(c)
    want_sha = []
    want = od.generate(prompt, c["new_tokens"], on_logits=lambda i, lg: want_sha.append(OD.sha_u16(lg)))
    _say("[gpu] decoder, two-layer W8 model: weights, eager steps")
    w, dec = _decoder({"config": c}, dev, hashes=True)
    assert w.quantized_sha == od.qsha
    assert not dec.fused_norm and w.layers[0]["qkv"][0].dtype == torch.int8
    shas = []
    toks = dec.generate(prompt, c["new_tokens"], on_logits=lambda i, lg: shas.append(OD.sha_u16(_bits(lg))))
    first = next((i for i, (a, b) in enumerate(zip(shas, want_sha)) if a != b), None)
    assert first is None, f"logits differ first at step {first}"
    assert toks == want
    _say("[gpu] decoder, two-layer W8 model: graph replay")
    dec2 = Q.Qwen3Decoder(w, max_positions=dec.max_pos, max_new_tokens=dec.max_new)
    assert dec2.generate(prompt, c["new_tokens"], graph=True) == want


def test_decoder_qwen3_1p7b_matches_reference(dev):
    """Config 4: Qwen3-1.7B W4A16 g128, 128-token prompt, 256 greedy tokens."""
    fx = _fixture("qwen3_1p7b")
    _say("[gpu] decoder Qwen3-1.7B: weights (generated and quantized on the device)")
    w, dec = _decoder(fx, dev, hashes=True)
    bad = [k for k in fx["quantized_sha"] if fx["quantized_sha"][k] != w.quantized_sha.get(k)]
    assert not bad, f"{len(bad)} quantized tensors differ from the reference quantizer's, e.g. {bad[:3]}"
    _say("[gpu] decoder Qwen3-1.7B: 256 tokens, graph replay")
    toks = dec.generate(fx["prompt"], len(fx["tokens"]), graph=True)
    if toks != fx["tokens"]:
        i = next(i for i in range(len(toks)) if toks[i] != fx["tokens"][i])
        lg = fx["logits"][i]
        pytest.fail(f"token {i} differs: {toks[i]} vs {fx['tokens'][i]} (reference top two {lg['top']})")
    _say("[gpu] decoder Qwen3-1.7B: eager steps, logits of the first 16 tokens")
    from pilm_amd import qwen3 as Q
    dec2 = Q.Qwen3Decoder(w, max_positions=dec.max_pos, max_new_tokens=dec.max_new)
    shas = []
    dec2.generate(fx["prompt"], 16, on_logits=lambda i, lg: shas.append(OD.sha_u16(_bits(lg))))
    assert shas == [lg["sha"] for lg in fx["logits"][:16]]
