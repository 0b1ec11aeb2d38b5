"""The quantized Linear modules and the SwiGLU fusion step on device tensors.

Mirrors piLM's src/models/base/linear.py:188-557 (`QuantizedW8A32Linear`,
`QuantizedW4A16Linear`, `QuantizedW8A32SwiGLU`, `QuantizedW4A16SwiGLU`) and
src/runtime/quantize.py:15-83 (`quantize_linear_modules_w8a32`,
`fuse_quantized_swiglu_modules`): the same buffers, constructor arguments,
reshape rules (1-D input -> one row and back, >2-D flattened to rows and
restored), kernel choice (bf16 input -> W8A16, otherwise fp32 W8A32 and a cast
back; W4 per-row / g128 / g32 by the scale shape) and errors. Buffers and
inputs live on the GPU; the kernels are the HIP library's, called through
pilm_amd.ckernel.

Differences, all on the device side:
  * the SwiGLU activation between the two linears reproduces torch's CPU
    `F.silu(gate) * up` bit for bit (PILM_SWIGLU_ACT_BACKEND=torch, the
    default, as in piLM; computed by ekernel_silu_mul_bf16, because torch's
    own GPU silu rounds differently) or is the library's bf16 SwiGLU
    (=ckernel, the reference's ekernel_swiglu_bf16);
  * the fused W4 SwiGLU kernel (one-row inputs) is opt-in with
    PILM_W4_SWIGLU_FUSED=1, as in piLM; it rounds silu(g) * u once, the
    default path rounds silu(g) to bf16 first.
"""
from __future__ import annotations

import os

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ckernel

_GPU = "cuda"


def _rows(input: torch.Tensor):
    """linear.py:211-221: (x2d, squeeze, original_shape)."""
    original_shape = tuple(input.shape)
    if input.ndim == 1:
        return input.reshape(1, -1), True, original_shape
    if input.ndim == 2:
        return input, False, original_shape
    return input.reshape(-1, input.shape[-1]), False, original_shape


def _unrows(out: torch.Tensor, squeeze: bool, original_shape) -> torch.Tensor:
    if squeeze:
        return out.reshape(-1)
    if len(original_shape) > 2:
        return out.reshape(*original_shape[:-1], out.shape[-1])
    return out


def _swiglu_act(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """linear.py:408-421 / 534-545: silu(gate) * up as torch computes it on
    the CPU (bf16), or the reference's bf16 SwiGLU kernel (=ckernel)."""
    if gate.dtype == torch.bfloat16 and gate.device.type == _GPU:
        if os.environ.get("PILM_SWIGLU_ACT_BACKEND", "torch").lower() == "ckernel":
            return ckernel.swiglu_bf16(gate, up)
        return ckernel.silu_mul_bf16(gate, up)
    return F.silu(gate) * up


def _w4_swiglu_fused_enabled() -> bool:
    """linear.py:43-49: the fused W4 SwiGLU kernel only with PILM_W4_SWIGLU_FUSED=1."""
    return os.environ.get("PILM_W4_SWIGLU_FUSED", "0") == "1"


class QuantizedW8A32Linear(nn.Module):
    """linear.py:188-264: int8 per-output-channel weights + fp32 scales."""

    def __init__(self, qweight: torch.Tensor, scales: torch.Tensor):
        super().__init__()
        self.register_buffer("qweight", qweight.contiguous())
        self.register_buffer("scales", scales.contiguous())
        self.in_features = qweight.shape[1]
        self.out_features = qweight.shape[0]

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> "QuantizedW8A32Linear":
        if linear.bias is not None:
            raise ValueError("QuantizedW8A32Linear only supports bias-free Linear")
        qweight, scales = ckernel.quantize_weight_i8_per_row(linear.weight.detach().to(torch.float32))
        return cls(qweight, scales)

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        if input.dtype == torch.bfloat16 and input.device.type == _GPU:
            x2d, squeeze, shape = _rows(input)
            return _unrows(ckernel.linear_w8a16_bf16(x2d, self.qweight, self.scales), squeeze, shape)
        original_dtype = input.dtype
        x2d, squeeze, shape = _rows(input.to(torch.float32))
        out = ckernel.linear_w8a32(x2d, self.qweight, self.scales)
        return _unrows(out, squeeze, shape).to(original_dtype)

    def argmax_bf16(self, input: torch.Tensor) -> int:
        """linear.py:260-264: greedy token of one bf16 row (lm_head)."""
        if input.dtype != torch.bfloat16 or input.device.type != _GPU:
            raise ValueError("argmax_bf16 requires GPU BF16 input")
        return ckernel.linear_w8a16_bf16_argmax(input, self.qweight, self.scales)


class QuantizedW4A16Linear(nn.Module):
    """linear.py:267-340: nibble-packed int4 weights; per-row scales [N]
    (bundle v2) or group scales [N, ceil(K/G)], G = 128 when the group count
    matches, else 32."""

    def __init__(self, qweight: torch.Tensor, scales: torch.Tensor, in_features: int):
        super().__init__()
        self.register_buffer("qweight", qweight.contiguous())
        self.register_buffer("scales", scales.contiguous())
        self.in_features = int(in_features)
        self.out_features = qweight.shape[0]
        self.group_size = None
        if scales.ndim == 2:
            groups = int(scales.shape[1])
            self.group_size = 128 if groups == (self.in_features + 127) // 128 else 32

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> "QuantizedW4A16Linear":
        if linear.bias is not None:
            raise ValueError("QuantizedW4A16Linear only supports bias-free Linear")
        qweight, scales = ckernel.quantize_weight_i4_per_row_chunked(linear.weight.detach().to(torch.float32))
        return cls(qweight, scales, linear.in_features)

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        if input.dtype != torch.bfloat16 or input.device.type != _GPU:
            raise ValueError("QuantizedW4A16Linear currently requires GPU BF16 input")
        x2d, squeeze, shape = _rows(input)
        if self.scales.ndim == 2:
            fn = ckernel.linear_w4a16g128_bf16 if self.group_size == 128 else ckernel.linear_w4a16g32_bf16
            out = fn(x2d, self.qweight, self.scales, self.in_features)
        else:
            out = ckernel.linear_w4a16_bf16(x2d, self.qweight, self.scales, self.in_features)
        return _unrows(out, squeeze, shape)


class QuantizedW8A32SwiGLU(nn.Module):
    """linear.py:343-432: gate and up as one int8 GEMV over their
    concatenated rows, the SwiGLU activation, then the down GEMV."""

    def __init__(self, gate_up_qweight, gate_up_scales, down_qweight, down_scales, intermediate_size: int):
        super().__init__()
        self.register_buffer("gate_up_qweight", gate_up_qweight.contiguous())
        self.register_buffer("gate_up_scales", gate_up_scales.contiguous())
        self.register_buffer("down_qweight", down_qweight.contiguous())
        self.register_buffer("down_scales", down_scales.contiguous())
        self.intermediate_size = intermediate_size

    @classmethod
    def from_swiglu(cls, swiglu: nn.Module) -> "QuantizedW8A32SwiGLU":
        if swiglu.gate.bias is not None or swiglu.up.bias is not None or swiglu.down.bias is not None:
            raise ValueError("QuantizedW8A32SwiGLU only supports bias-free Linear")
        q = ckernel.quantize_weight_i8_per_row
        gate_q, gate_s = q(swiglu.gate.weight.detach().to(torch.float32))
        up_q, up_s = q(swiglu.up.weight.detach().to(torch.float32))
        down_q, down_s = q(swiglu.down.weight.detach().to(torch.float32))
        return cls(torch.cat([gate_q, up_q], dim=0), torch.cat([gate_s, up_s], dim=0), down_q, down_s,
                   gate_q.shape[0])

    def _linear(self, x2d, qweight, scales):
        if x2d.dtype == torch.bfloat16:
            return ckernel.linear_w8a16_bf16(x2d, qweight, scales)
        return ckernel.linear_w8a32(x2d.to(torch.float32), qweight, scales).to(x2d.dtype)

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        x2d, squeeze, shape = _rows(input)
        gate_up = self._linear(x2d, self.gate_up_qweight, self.gate_up_scales)
        gate, up = gate_up.split(self.intermediate_size, dim=-1)
        hidden = _swiglu_act(gate.contiguous(), up.contiguous())
        return _unrows(self._linear(hidden, self.down_qweight, self.down_scales), squeeze, shape)


class QuantizedW4A16SwiGLU(nn.Module):
    """linear.py:435-557: per-row W4 gate_up [2I, ceil(K/2)] + down; one-row
    inputs take the fused kernel (gate_up -> bf16 SwiGLU -> down)."""

    def __init__(self, gate_up_qweight, gate_up_scales, down_qweight, down_scales, intermediate_size: int,
                 gate_up_in_features: int, down_in_features: int):
        super().__init__()
        self.register_buffer("gate_up_qweight", gate_up_qweight.contiguous())
        self.register_buffer("gate_up_scales", gate_up_scales.contiguous())
        self.register_buffer("down_qweight", down_qweight.contiguous())
        self.register_buffer("down_scales", down_scales.contiguous())
        self.intermediate_size = int(intermediate_size)
        self.gate_up_in_features = int(gate_up_in_features)
        self.down_in_features = int(down_in_features)

    def _linear(self, x2d, qweight, scales, in_features):
        if x2d.dtype != torch.bfloat16:
            raise ValueError("QuantizedW4A16SwiGLU requires GPU BF16 input")
        if scales.ndim != 1:
            raise ValueError("QuantizedW4A16SwiGLU currently supports per-row W4 scales only")
        return ckernel.linear_w4a16_bf16(x2d, qweight, scales, in_features)

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        x2d, squeeze, shape = _rows(input)
        if _w4_swiglu_fused_enabled() and x2d.shape[0] == 1 and x2d.dtype == torch.bfloat16:
            out = ckernel.swiglu_w4a16_bf16(x2d, self.gate_up_qweight, self.gate_up_scales, self.down_qweight,
                                            self.down_scales, self.intermediate_size, self.gate_up_in_features,
                                            self.down_in_features)
            return _unrows(out, squeeze, shape)
        gate_up = self._linear(x2d, self.gate_up_qweight, self.gate_up_scales, self.gate_up_in_features)
        gate, up = gate_up.split(self.intermediate_size, dim=-1)
        hidden = _swiglu_act(gate.contiguous(), up.contiguous())
        out = self._linear(hidden, self.down_qweight, self.down_scales, self.down_in_features)
        return _unrows(out, squeeze, shape)


class SwiGLU(nn.Module):
    """The MLP block the fusion step looks for: bias-free gate, up and down
    projections, down(silu(gate(x)) * up(x)) (src/models/base/layers.py)."""

    def __init__(self, hidden_size: int, intermediate_size: int):
        super().__init__()
        self.gate = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.up = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.down = nn.Linear(intermediate_size, hidden_size, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down(F.silu(self.gate(x)) * self.up(x))


def quantize_linear_modules_w8a32(module: nn.Module, skip_lm_head: bool = True, prefix: str = "") -> int:
    """quantize.py:15-30: replace bias-free Linear children by
    QuantizedW8A32Linear in place (lm_head kept unless skip_lm_head=False)."""
    replaced = 0
    for name, child in list(module.named_children()):
        child_prefix = f"{prefix}.{name}" if prefix else name
        if skip_lm_head and child_prefix == "lm_head":
            continue
        if isinstance(child, nn.Linear) and child.bias is None:
            setattr(module, name, QuantizedW8A32Linear.from_linear(child))
            replaced += 1
        else:
            replaced += quantize_linear_modules_w8a32(child, skip_lm_head=skip_lm_head, prefix=child_prefix)
    return replaced


def fuse_quantized_swiglu_modules(module: nn.Module) -> int:
    """quantize.py:33-83: replace SwiGLU blocks whose gate, up and down are
    already quantized (all W8, or all per-row W4) by the fused modules, gate
    rows first in the concatenated [2I, ...] matrix.  Returns the count."""
    fused = 0
    for name, child in list(module.named_children()):
        if isinstance(child, SwiGLU) and all(isinstance(getattr(child, p), QuantizedW8A32Linear)
                                            for p in ("gate", "up", "down")):
            setattr(module, name, QuantizedW8A32SwiGLU(
                gate_up_qweight=torch.cat([child.gate.qweight, child.up.qweight], dim=0),
                gate_up_scales=torch.cat([child.gate.scales, child.up.scales], dim=0),
                down_qweight=child.down.qweight, down_scales=child.down.scales,
                intermediate_size=child.gate.out_features))
            fused += 1
        elif (isinstance(child, SwiGLU)
              and all(isinstance(getattr(child, p), QuantizedW4A16Linear) for p in ("gate", "up", "down"))
              and all(getattr(child, p).scales.ndim == 1 for p in ("gate", "up", "down"))):
            setattr(module, name, QuantizedW4A16SwiGLU(
                gate_up_qweight=torch.cat([child.gate.qweight, child.up.qweight], dim=0),
                gate_up_scales=torch.cat([child.gate.scales, child.up.scales], dim=0),
                down_qweight=child.down.qweight, down_scales=child.down.scales,
                intermediate_size=child.gate.out_features,
                gate_up_in_features=child.gate.in_features,
                down_in_features=child.down.in_features))
            fused += 1
        else:
            fused += fuse_quantized_swiglu_modules(child)
    return fused
