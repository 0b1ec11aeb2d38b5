"""CPU: the decoder-step oracle (oracle/decoder.c) against torch and against
the reference's own fixtures.

The oracle restates the orders and functions torch's CPU kernels use for the
torch steps of piLM's decoder layer.  Two kinds of pin:
  * torch itself, black box, on the operations the reference's lines call
    (torch.sum / mean, softmax, sigmoid, silu, rsqrt, bf16 bmm), with the
    fixtures' settings (AVX2 kernels, oneDNN off) -- designed inputs reveal
    the summation trees (cancelling +-2^40 pairs count the addends outside
    the pair's subtree), random inputs check the rest bit for bit;
  * the reference: the oracle decoder (oracle/decoder.py) built from these
    steps, the linear oracle and the quantizer restatement must reproduce
    the fixture piLM's Engine.generate wrote (tests/golden/decode_tiny.json):
    every quantized tensor's hash, the rope tables' hash, every step's full
    bf16 logits and the 48 greedy tokens.  An attention output one bf16 ulp
    off must fail that comparison.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import decoder as OD
from pilm_amd import synth as S
from tests.conftest import torch_cpu_like_fixture

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def torch():
    return torch_cpu_like_fixture()


def _bf16_bits(t):
    import torch as _t
    return t.to(_t.bfloat16).view(_t.int16).numpy().view(np.uint16)


# ----------------------------------------------------------------- sums

@pytest.mark.parametrize("n", [32, 100, 128, 300, 2048, 3000, 4096, 6144, 12288])
def test_torch_sum_order(torch, n):
    rng = np.random.default_rng(n)
    for _ in range(40):
        x = (rng.standard_normal(n) * np.exp(rng.standard_normal(n) * 3)).astype(np.float32)
        assert OD.torch_sum(x) == np.float32(torch.from_numpy(x).sum().item())


def test_torch_sum_tree_revealed(torch):
    """+-2^40 at i and j, ones elsewhere: the sum counts the ones outside the
    smallest subtree holding both, which fixes the tree."""
    n = 2048
    for i, j in [(0, 8), (0, 32), (0, 512), (5, 37), (100, 1900), (7, 15), (0, 2047)]:
        x = np.ones(n, np.float32)
        x[i], x[j] = 2.0 ** 40, -(2.0 ** 40)
        assert OD.torch_sum(x) == np.float32(torch.from_numpy(x).sum().item()), (i, j)


def test_mean_is_sum_over_n(torch):
    rng = np.random.default_rng(1)
    for n in (128, 2048, 100, 3000):
        x = S.bf16_bits_to_f32(S.f32_to_bf16_bits(rng.standard_normal(n).astype(np.float32)))
        t = torch.from_numpy(x).pow(2).mean(-1, keepdim=True).item()
        assert np.float32(t) == np.float32(OD.torch_sum(x * x) / np.float32(n))


# ------------------------------------------------------- exp, softmax, acts

def test_sleef_exp_is_softmax_exp(torch):
    """softmax([0, d]) for d < -17 returns exp(d) itself (1 + exp(d) rounds to 1)."""
    d = -np.linspace(17, 103, 50001).astype(np.float32)
    rows = np.stack([np.zeros_like(d), d], 1)
    got = torch.softmax(torch.from_numpy(rows), dim=-1).numpy()[:, 1]
    assert np.array_equal(got.view(np.uint32), OD.sleef_expf(d).view(np.uint32))


def test_sleef_exp_within_one_ulp():
    x = np.linspace(-100, 80, 400001).astype(np.float32)
    ref = np.exp(x.astype(np.float64))
    got = OD.sleef_expf(x).astype(np.float64)
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - ref) <= ulp)


@pytest.mark.parametrize("n", [1, 3, 7, 8, 9, 16, 17, 100, 129, 384, 1000])
def test_softmax_rows(torch, n):
    rng = np.random.default_rng(n)
    x = S.bf16_bits_to_f32(S.f32_to_bf16_bits((rng.standard_normal((30, n)) * 3).astype(np.float32)))
    x[0, :] = 0.0                                 # all equal
    got = torch.softmax(torch.from_numpy(x.copy()), dim=-1).numpy()
    assert np.array_equal(got.view(np.uint32), OD.softmax_f32(x).view(np.uint32))


def test_sigmoid_and_silu_every_bf16(torch):
    import torch as T
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    xb = T.from_numpy(bits.view(np.int16)).view(T.bfloat16)
    fin = np.isfinite(S.bf16_bits_to_f32(bits))
    sig = T.sigmoid(xb).view(T.int16).numpy().view(np.uint16)
    slu = T.nn.functional.silu(xb).view(T.int16).numpy().view(np.uint16)
    assert np.array_equal(sig[fin], OD.sigmoid_bf16(bits)[fin])
    assert np.array_equal(slu[fin], OD.silu_bf16(bits)[fin])


# ------------------------------------------------------------ layer steps

def _gemma(torch, x, w, eps):
    """GemmaRMSNorm.forward's operations (layers.py:142-147) in torch."""
    orig = x.dtype
    xf = x.to(torch.float32)
    var = xf.pow(2).mean(-1, keepdim=True)
    xf = xf * torch.rsqrt(var + eps)
    return (w + 1.0) * xf.to(orig)


@pytest.mark.parametrize("rows,n", [(1, 2048), (16, 2048), (3, 4096), (2, 128), (5, 296)])
def test_rmsnorm_against_torch(torch, rows, n):
    rng = np.random.default_rng(rows * n)
    x = torch.from_numpy(rng.standard_normal((rows, n)).astype(np.float32) * 3).to(torch.bfloat16)
    r = torch.from_numpy(rng.standard_normal((rows, n)).astype(np.float32)).to(torch.bfloat16)
    w = torch.from_numpy(rng.standard_normal(n).astype(np.float32) * 0.02).to(torch.bfloat16)
    h = r + x
    want = _bf16_bits(_gemma(torch, h, w, 1e-6))
    out, res_out = OD.rmsnorm_gemma_bf16(_bf16_bits(x), _bf16_bits(r), _bf16_bits(w), 1e-6)
    assert np.array_equal(res_out, _bf16_bits(h))
    assert np.array_equal(out, want)
    out2, _ = OD.rmsnorm_gemma_bf16(_bf16_bits(x), None, _bf16_bits(w), 1e-6)
    assert np.array_equal(out2, _bf16_bits(_gemma(torch, x, w, 1e-6)))


def _rope(torch, q, k, cos, sin, rot):
    """apply_rope's operations (layers.py:150-195) for q, k [seq, heads, D]."""
    nf = rot // 2
    cb, sb = cos.unsqueeze(1), sin.unsqueeze(1)
    out = []
    for t in (q, k):
        tr = t[..., :rot].to(torch.float32)
        a, b = tr[..., :nf], tr[..., nf:]
        r = torch.cat([a * cb - b * sb, a * sb + b * cb], dim=-1)
        out.append(torch.cat([r.to(t.dtype), t[..., rot:]], dim=-1))
    return out


def _attention(torch, q, full_k, full_v, gate, n_heads, n_kv, is_decode):
    """FullAttention.forward's operations after the cache gather
    (attention.py:117-139); q [S, H, D] roped, full_k / full_v [L, Hkv, D]."""
    seq, _, D = q.shape
    if n_kv < n_heads:
        rep = n_heads // n_kv
        full_k = full_k.unsqueeze(2).expand(-1, -1, rep, -1).reshape(full_k.shape[0], n_heads, D)
        full_v = full_v.unsqueeze(2).expand(-1, -1, rep, -1).reshape(full_v.shape[0], n_heads, D)
    qq, k_t, v_t = q.transpose(0, 1), full_k.transpose(0, 1), full_v.transpose(0, 1)
    scores = torch.bmm(qq, k_t.transpose(1, 2)) * (1.0 / math.sqrt(D))
    if not is_decode or seq > 1:
        kv_len = full_k.shape[0]
        mask = torch.triu(torch.ones(seq, kv_len, dtype=torch.bool), diagonal=kv_len - seq + 1)
        scores = scores.masked_fill(mask.unsqueeze(0), float("-inf"))
    attn = torch.softmax(scores.to(torch.float32), dim=-1).to(v_t.dtype)
    out = torch.bmm(attn, v_t).transpose(0, 1).reshape(seq, -1)
    return out * torch.sigmoid(gate) if gate is not None else out


@pytest.mark.parametrize("S,H,Hkv,D,pos0", [(1, 16, 8, 128, 200), (16, 16, 8, 128, 32), (5, 4, 2, 128, 11),
                                            (3, 8, 8, 64, 0), (2, 4, 1, 256, 40)])
def test_qk_rope_and_attention_against_torch(torch, S, H, Hkv, D, pos0):
    rng = np.random.default_rng(S * 1000 + pos0)
    bs, L = 16, pos0 + S
    nblk = (L + bs - 1) // bs + 1
    block_ids = rng.permutation(nblk + 3)[:nblk].astype(np.int32)        # scattered physical blocks
    kc = np.zeros((nblk + 3, bs, Hkv, D), np.uint16)
    vc = np.zeros_like(kc)
    old_k = torch.from_numpy(rng.standard_normal((pos0, Hkv, D)).astype(np.float32)).to(torch.bfloat16)
    old_v = torch.from_numpy(rng.standard_normal((pos0, Hkv, D)).astype(np.float32)).to(torch.bfloat16)
    for j in range(pos0):
        kc[block_ids[j // bs], j % bs] = _bf16_bits(old_k[j])
        vc[block_ids[j // bs], j % bs] = _bf16_bits(old_v[j])
    qg = torch.from_numpy(rng.standard_normal((S, H, 2 * D)).astype(np.float32)).to(torch.bfloat16)
    k = torch.from_numpy(rng.standard_normal((S, Hkv, D)).astype(np.float32)).to(torch.bfloat16)
    v = torch.from_numpy(rng.standard_normal((S, Hkv, D)).astype(np.float32)).to(torch.bfloat16)
    qw = torch.from_numpy(rng.standard_normal(D).astype(np.float32) * 0.02).to(torch.bfloat16)
    kw = torch.from_numpy(rng.standard_normal(D).astype(np.float32) * 0.02).to(torch.bfloat16)
    cos, sin = OD.rope_tables(1e6, D, L + 1)
    # torch side: attention.py:82-139 on the same numbers
    qs, gate = torch.chunk(qg, 2, dim=-1)
    gate = gate.reshape(S, -1)
    qn, kn = _gemma(torch, qs, qw, 1e-6), _gemma(torch, k, kw, 1e-6)
    qr, kr = _rope(torch, qn, kn, torch.from_numpy(cos[pos0:L]), torch.from_numpy(sin[pos0:L]), D)
    full_k, full_v = torch.cat([old_k, kr]), torch.cat([old_v, v])
    want = _attention(torch, qr, full_k, full_v, gate, H, Hkv, is_decode=S == 1)
    # oracle side
    q_out = OD.qk_norm_rope_bf16(_bf16_bits(qg).reshape(S, -1), _bf16_bits(k).reshape(S, -1),
                                 _bf16_bits(v).reshape(S, -1), _bf16_bits(qw), _bf16_bits(kw), cos, sin, pos0, kc, vc,
                                 block_ids, n_heads=H, n_kv_heads=Hkv, head_dim=D, rot_dim=D, eps=1e-6, block_size=bs)
    assert np.array_equal(q_out, _bf16_bits(qr))
    for s in range(S):
        j = pos0 + s
        assert np.array_equal(kc[block_ids[j // bs], j % bs], _bf16_bits(kr[s]))
        assert np.array_equal(vc[block_ids[j // bs], j % bs], _bf16_bits(v[s]))
    gate_bits = _bf16_bits(qg).reshape(-1)[D:]
    got = OD.attention_exact_bf16(q_out, kc, vc, block_ids, L, gate_bits, H * 2 * D, 2 * D, block_size=bs)
    assert np.array_equal(got, _bf16_bits(want))


@pytest.mark.parametrize("L", [1, 2, 3, 4])
def test_attention_small_kernel_orders(torch, L):
    """Decode over 1-4 positions: torch's small-matrix kernel (S*L*D < 400)
    below four positions, the blocked kernels from it."""
    rng = np.random.default_rng(L)
    H, Hkv, D, bs = 2, 1, 128, 16
    q = torch.from_numpy(rng.standard_normal((1, H, D)).astype(np.float32) * 4).to(torch.bfloat16)
    kk = torch.from_numpy(rng.standard_normal((L, Hkv, D)).astype(np.float32) * 4).to(torch.bfloat16)
    vv = torch.from_numpy(rng.standard_normal((L, Hkv, D)).astype(np.float32)).to(torch.bfloat16)
    kc = np.zeros((1, bs, Hkv, D), np.uint16)
    vc = np.zeros_like(kc)
    kc[0, :L], vc[0, :L] = _bf16_bits(kk), _bf16_bits(vv)
    want = _attention(torch, q, kk, vv, None, H, Hkv, True)
    got = OD.attention_exact_bf16(_bf16_bits(q), kc, vc, np.zeros(1, np.int32), L, block_size=bs)
    assert np.array_equal(got, _bf16_bits(want))


# ------------------------------------------------------- the reference itself

def _fixture(name):
    return json.loads((GOLDEN / f"decode_{name}.json").read_text())


def test_fixture_records_the_reference_settings():
    fx = _fixture("tiny")
    g = fx["generated_with"]
    assert g["cpu_capability"] == "AVX2" and g["mkldnn"] is False
    assert len(fx["tokens"]) == fx["config"]["new_tokens"] == len(fx["logits"])
    assert [lg["argmax"] for lg in fx["logits"]] == fx["tokens"]


def test_oracle_decoder_reproduces_reference_fixture():
    """Every quantized tensor, the rope tables, every step's bf16 logits and
    all greedy tokens equal what piLM's engine wrote."""
    fx = _fixture("tiny")
    dec = OD.OracleDecoder(fx["config"])
    assert dec.qsha == fx["quantized_sha"]
    import hashlib
    cos, sin = OD.rope_tables(fx["config"]["rope_theta"], dec.rot, fx["rope"]["positions"])
    assert hashlib.sha256(cos.tobytes()).hexdigest() == fx["rope"]["cos_sha"]
    assert hashlib.sha256(sin.tobytes()).hexdigest() == fx["rope"]["sin_sha"]
    shas = []
    toks = dec.generate(fx["prompt"], len(fx["tokens"]), lambda i, lg: shas.append(OD.sha_u16(lg)))
    assert shas == [lg["sha"] for lg in fx["logits"]]
    assert toks == fx["tokens"]


def test_perturbed_oracle_misses_the_fixture(monkeypatch):
    """The fixture rejects the smallest attention mistake: every attention
    output one bf16 ulp off once the context passes 40 positions changes the
    logits of the first generated tokens."""
    fx = _fixture("tiny")
    real = OD.attention_exact_bf16

    def one_ulp_off(q, k_cache, v_cache, block_ids, cache_len, gate=None, gate_row_stride=0, gate_head_stride=0,
                    *, block_size):
        out = real(q, k_cache, v_cache, block_ids, cache_len, gate, gate_row_stride, gate_head_stride,
                   block_size=block_size)
        return out ^ np.uint16(1) if cache_len > 40 else out
    monkeypatch.setattr(OD, "attention_exact_bf16", one_ulp_off)
    dec = OD.OracleDecoder(fx["config"])
    shas = []
    dec.generate(fx["prompt"], 8, lambda i, lg: shas.append(OD.sha_u16(lg)))
    assert shas != [lg["sha"] for lg in fx["logits"][:8]]


def test_device_quantizer_matches_reference_quantizer_on_cpu():
    """pilm_amd.ckernel's grouped int4 quantizer (the one the device decoder
    runs on the GPU) on the CPU gives the bytes of the reference's
    quantize_weight_i4_grouped_chunked, as hashed in the fixture."""
    import hashlib
    import torch as T
    from pilm_amd import ckernel as ck
    from pilm_amd import synth_model as SM
    fx = _fixture("tiny")
    c = fx["config"]
    ids = SM.tensor_ids(c["layers"])
    for name in ("layers.0.self_attn.q_proj", "layers.0.mlp.gate", "layers.1.self_attn.v_proj", "lm_head"):
        dims = {"q_proj": (2 * c["heads"] * c["head_dim"], c["hidden"]), "gate": (c["intermediate"], c["hidden"]),
                "v_proj": (c["kv_heads"] * c["head_dim"], c["hidden"]), "lm_head": (c["vocab"], c["hidden"])}
        shape = dims[name.split(".")[-1]]
        w = SM.normal_f32(c["seed"], ids[name], shape, c["std"])
        q, s = ck.quantize_weight_i4_grouped_chunked(w, group_size=128, rows_per_chunk=1000)
        got = [hashlib.sha256(q.numpy().tobytes()).hexdigest(), hashlib.sha256(s.numpy().tobytes()).hexdigest()]
        assert got == fx["quantized_sha"][name], name
        assert q.dtype == T.uint8
