"""The quantized Linear modules and the SwiGLU fusion step (pilm_amd.linear),
mirrors of piLM's linear.py / quantize.py: module structure and dispatch on
the CPU (no kernel call), forward parity on the GPU through the C ABI."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")
nn = torch.nn

from oracle import oracle as O  # noqa: E402
from pilm_amd import linear as L  # noqa: E402
from pilm_amd import synth as S  # noqa: E402
from tests import _golden as GV  # noqa: E402


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


# ------------------------------------------------------------------ CPU

def test_w4_group_size_from_scale_shape():
    q = torch.zeros((8, 150), dtype=torch.uint8)
    assert L.QuantizedW4A16Linear(q, torch.ones(8), 300).group_size is None
    assert L.QuantizedW4A16Linear(q, torch.ones(8, 3), 300).group_size == 128     # ceil(300/128) = 3
    assert L.QuantizedW4A16Linear(q, torch.ones(8, 10), 300).group_size == 32     # ceil(300/32) = 10
    m = L.QuantizedW4A16Linear(q, torch.ones(8), 300)
    assert (m.in_features, m.out_features) == (300, 8)


def test_rows_reshape_rules():
    for shape, rows in (((5,), (1, 5)), ((3, 5), (3, 5)), ((2, 3, 5), (6, 5))):
        x = torch.zeros(shape)
        x2d, squeeze, orig = L._rows(x)
        assert tuple(x2d.shape) == rows
        out = torch.zeros((x2d.shape[0], 7))
        assert tuple(L._unrows(out, squeeze, orig).shape) == tuple(shape[:-1]) + (7,)


def test_quantize_and_fuse_module_tree():
    torch.manual_seed(0)

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj = nn.Linear(16, 16, bias=False)
            self.biased = nn.Linear(16, 4, bias=True)
            self.mlp = L.SwiGLU(16, 24)

    class Model(nn.Module):
        def __init__(self):
            super().__init__()
            self.layers = nn.ModuleList([Block(), Block()])
            self.lm_head = nn.Linear(16, 40, bias=False)

    model = Model()
    gate_w = model.layers[0].mlp.gate.weight.detach().clone()
    # 2 blocks x (q_proj + gate/up/down); lm_head skipped, biased Linear kept
    assert L.quantize_linear_modules_w8a32(model) == 8
    assert isinstance(model.lm_head, nn.Linear) and isinstance(model.layers[0].biased, nn.Linear)
    mlp = model.layers[0].mlp
    gq, gs = O.quantize_weight_i8_per_row(gate_w.numpy())
    assert np.array_equal(mlp.gate.qweight.numpy(), gq) and np.array_equal(mlp.gate.scales.numpy(), gs)
    gate_q, up_q = mlp.gate.qweight.clone(), mlp.up.qweight.clone()
    assert L.fuse_quantized_swiglu_modules(model) == 2
    fused = model.layers[0].mlp
    assert isinstance(fused, L.QuantizedW8A32SwiGLU) and fused.intermediate_size == 24
    assert torch.equal(fused.gate_up_qweight, torch.cat([gate_q, up_q]))       # gate rows first
    assert tuple(fused.gate_up_scales.shape) == (48,)


def test_fuse_w4_per_row_only():
    def w4(n, k, grouped=False):
        q = torch.zeros((n, (k + 1) // 2), dtype=torch.uint8)
        return L.QuantizedW4A16Linear(q, torch.ones(n, (k + 127) // 128) if grouped else torch.ones(n), k)

    class M(nn.Module):
        def __init__(self, grouped):
            super().__init__()
            self.mlp = L.SwiGLU(16, 24)
            self.mlp.gate, self.mlp.up, self.mlp.down = w4(24, 16, grouped), w4(24, 16, grouped), w4(16, 24, grouped)

    m = M(False)
    assert L.fuse_quantized_swiglu_modules(m) == 1
    f = m.mlp
    assert isinstance(f, L.QuantizedW4A16SwiGLU)
    assert (f.intermediate_size, f.gate_up_in_features, f.down_in_features) == (24, 16, 24)
    assert tuple(f.gate_up_qweight.shape) == (48, 8)
    assert L.fuse_quantized_swiglu_modules(M(True)) == 0     # group scales stay unfused, as in piLM


def test_modules_reject_cpu_input():
    m = L.QuantizedW4A16Linear(torch.zeros((8, 8), dtype=torch.uint8), torch.ones(8), 16)
    with pytest.raises(ValueError):
        m(torch.zeros((1, 16), dtype=torch.bfloat16))
    w8 = L.QuantizedW8A32Linear(torch.zeros((8, 16), dtype=torch.int8), torch.ones(8))
    with pytest.raises(ValueError):
        w8.argmax_bf16(torch.zeros((16,), dtype=torch.bfloat16))


# ------------------------------------------------------------------ GPU

def _dev_bf16(bits: np.ndarray, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(torch.bfloat16)


def _bits(t) -> np.ndarray:
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.gpu
def test_w8_module_forward_and_argmax(dev):
    n, k = 300, 512
    w = S.weights_i8(11, n, k)
    s = S.scales_uniform(12, (n,), fp16_round=False)
    mod = L.QuantizedW8A32Linear(torch.from_numpy(w), torch.from_numpy(s)).to(dev)
    xf = S.activations_f32(13, 6, k)
    _say("[gpu] W8A32 module fp32 3-D")
    y = mod(torch.from_numpy(xf).to(dev).reshape(2, 3, k))
    assert tuple(y.shape) == (2, 3, n)
    assert np.array_equal(y.reshape(6, n).cpu().numpy(), O.linear_w8a32(xf, w, s))
    xb = S.activations_bf16(14, 1, k)
    _say("[gpu] W8A16 module bf16 1-D + argmax")
    y = mod(_dev_bf16(xb, dev).reshape(-1))
    assert tuple(y.shape) == (n,) and np.array_equal(_bits(y), O.linear_w8a16_bf16(xb, w, s)[0])
    assert mod.argmax_bf16(_dev_bf16(xb, dev)) == O.linear_w8a16_bf16_argmax(xb, w, s)[0]


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["row", "g128", "g32"])
def test_w4_module_forward(kind, dev):
    n, k = 200, 768
    w = S.weights_i4_packed(21, n, k)
    g = {"row": 0, "g128": 128, "g32": 32}[kind]
    s = S.scales_uniform(22, (n,) if not g else (n, (k + g - 1) // g), fp16_round=False)
    mod = L.QuantizedW4A16Linear(torch.from_numpy(w), torch.from_numpy(s), k).to(dev)
    x = S.activations_bf16(23, 5, k)
    _say(f"[gpu] W4 module {kind}")
    y = mod(_dev_bf16(x, dev))
    ref = O.linear_w4a16_bf16(x, w, s) if not g else O.linear_w4a16g_bf16(x, w, s, g)
    assert np.array_equal(_bits(y), ref)


def _w4_swiglu(dev, h=256, i=512):
    x, gu, gs, dw, ds = GV._gen().make_swiglu_inputs(h, i, h, 31)
    mod = L.QuantizedW4A16SwiGLU(torch.from_numpy(gu), torch.from_numpy(gs), torch.from_numpy(dw),
                                 torch.from_numpy(ds), i, h, i).to(dev)
    return mod, (x, gu, gs, dw, ds), i


@pytest.mark.gpu
def test_w4_swiglu_module_default_is_reference_default(dev, monkeypatch):
    """Unset switches: piLM's default path (linear.py:43-49, 534-545) --
    gate_up GEMV, torch's CPU silu(gate) * up in bf16, down GEMV -- for one
    row and for several, bit for bit."""
    from oracle import decoder as OD
    monkeypatch.delenv("PILM_W4_SWIGLU_FUSED", raising=False)
    monkeypatch.delenv("PILM_SWIGLU_ACT_BACKEND", raising=False)
    mod, (x, gu, gs, dw, ds), i = _w4_swiglu(dev)
    xs = np.concatenate([x, S.activations_bf16(33, 2, x.shape[1])])
    _say("[gpu] W4 SwiGLU module, default path")
    for rows in (xs[:1], xs):
        y = _bits(mod(_dev_bf16(rows, dev)))
        g_u = O.linear_w4a16_bf16(rows, gu, gs)
        act = OD.silu_mul_bf16(g_u[:, :i], g_u[:, i:], rows.shape[0], i, i)
        assert np.array_equal(y, O.linear_w4a16_bf16(act, dw, ds))


@pytest.mark.gpu
def test_w4_swiglu_module_fused_and_unfused(dev, monkeypatch):
    mod, ins, i = _w4_swiglu(dev)
    x = ins[0]
    monkeypatch.setenv("PILM_W4_SWIGLU_FUSED", "1")
    _say("[gpu] W4 SwiGLU module, one row (fused kernel)")
    assert np.array_equal(_bits(mod(_dev_bf16(x, dev).reshape(-1))), O.swiglu_w4a16_bf16(*ins, i)[0])
    # unfused with the library's SwiGLU activation: the same bits, row by row
    monkeypatch.setenv("PILM_W4_SWIGLU_FUSED", "0")
    monkeypatch.setenv("PILM_SWIGLU_ACT_BACKEND", "ckernel")
    xs = np.concatenate([x, S.activations_bf16(32, 2, x.shape[1])])
    _say("[gpu] W4 SwiGLU module, three rows (unfused, ckernel activation)")
    y = _bits(mod(_dev_bf16(xs, dev)))
    for r in range(3):
        assert np.array_equal(y[r], O.swiglu_w4a16_bf16(xs[r:r + 1], *ins[1:], i)[0]), r


@pytest.mark.gpu
def test_w8_swiglu_module_matches_composition(dev, monkeypatch):
    monkeypatch.setenv("PILM_SWIGLU_ACT_BACKEND", "ckernel")
    h, i = 256, 384
    gw, uw, dw = (S.weights_i8(40 + j, r, c) for j, (r, c) in enumerate(((i, h), (i, h), (h, i))))
    gs, us, ds = (S.scales_uniform(50 + j, (r,), fp16_round=False) for j, r in enumerate((i, i, h)))
    mod = L.QuantizedW8A32SwiGLU(torch.from_numpy(np.concatenate([gw, uw])),
                                 torch.from_numpy(np.concatenate([gs, us])),
                                 torch.from_numpy(dw), torch.from_numpy(ds), i).to(dev)
    x = S.activations_bf16(60, 2, h)
    _say("[gpu] W8 SwiGLU module")
    y = _bits(mod(_dev_bf16(x, dev)))
    g = O.linear_w8a16_bf16(x, gw, gs)
    u = O.linear_w8a16_bf16(x, uw, us)
    hid = O.swiglu_bf16(g, u)
    assert np.array_equal(y, O.linear_w8a16_bf16(hid, dw, ds))
