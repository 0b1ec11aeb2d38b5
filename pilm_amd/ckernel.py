"""torch-tensor wrappers around the HIP libecpu, plus the weight quantizers.

Mirrors src/runtime/ckernel.py of piLM: the same function names, argument
meaning, dtype/ndim/shape rules and error behaviour (ValueError for a bad
argument, RuntimeError("ekernel_... failed: rc=...") for a nonzero C return
code).  The difference is residency: kernel inputs must be GPU tensors
(PyTorch-ROCm reports them as device type "cuda"), outputs are allocated on
the same device, and work is enqueued on PyTorch's current stream.

The quantizers (ckernel.py:70-161) and the int4 unpack helper (:279-296)
produce/consume the reference's packed layout and run on whatever device the
weight lives on.
"""
from __future__ import annotations

import ctypes
from typing import Tuple

import torch

from . import bindings as abi

_GPU = "cuda"   # PyTorch-ROCm names HIP devices "cuda"


def _bind_stream(t: torch.Tensor) -> None:
    abi.set_stream(torch.cuda.current_stream(t.device).cuda_stream)


def _rc_error(name: str, rc: int) -> RuntimeError:
    err = abi.last_error()
    return RuntimeError(f"{name} failed: rc={rc}" + (f" ({err})" if err else ""))


def _require_f32_gpu_2d(name: str, tensor: torch.Tensor) -> torch.Tensor:
    if tensor.device.type != _GPU:
        raise ValueError(f"{name} must be a GPU tensor")
    if tensor.dtype != torch.float32:
        raise ValueError(f"{name} must be torch.float32, got {tensor.dtype}")
    if tensor.ndim != 2:
        raise ValueError(f"{name} must be 2D, got shape={tuple(tensor.shape)}")
    return tensor.contiguous()


def _same_device(*ts: torch.Tensor) -> None:
    devs = {t.device for t in ts}
    if len(devs) != 1:
        raise ValueError(f"all tensors must be on one device, got {sorted(map(str, devs))}")


# ------------------------------------------------------------------ GEMM

def gemm_f32(a: torch.Tensor, b: torch.Tensor, transpose_b: bool = False) -> torch.Tensor:
    """ckernel.py:23-46: a[M,K] @ b[K,N] (or b[N,K].T when transpose_b)."""
    a = _require_f32_gpu_2d("a", a)
    b = _require_f32_gpu_2d("b", b)
    _same_device(a, b)
    m, k = a.shape
    if transpose_b:
        n, kb = b.shape
    else:
        kb, n = b.shape
    if kb != k:
        raise ValueError(f"incompatible GEMM shapes: a={tuple(a.shape)} b={tuple(b.shape)} transpose_b={transpose_b}")
    out = torch.empty((m, n), dtype=torch.float32, device=a.device)
    _bind_stream(a)
    desc = abi.EkernelGemmDesc(m, n, k, abi.ECPU_PRECISION_F32, abi.ECPU_PRECISION_F32, abi.ECPU_PRECISION_F32,
                               0, int(transpose_b))
    lib = abi._load_lib()
    rc = lib.ekernel_gemm(ctypes.byref(desc), ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr()),
                          ctypes.c_void_p(out.data_ptr()), lib.ekernel_detect_isa())
    if rc != 0:
        raise _rc_error("ekernel_gemm", rc)
    return out


def _as_2d(x: torch.Tensor):
    original_shape: Tuple[int, ...] = tuple(x.shape)
    if x.ndim == 1:
        return x.reshape(1, -1), True, original_shape
    if x.ndim == 2:
        return x, False, original_shape
    return x.reshape(-1, x.shape[-1]), False, original_shape


def _restore(out: torch.Tensor, squeeze: bool, original_shape) -> torch.Tensor:
    if squeeze:
        return out.reshape(-1)
    if len(original_shape) > 2:
        return out.reshape(*original_shape[:-1], out.shape[-1])
    return out


def linear_f32(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """ckernel.py:49-67: F32 linear without bias, x @ weight.T."""
    x2d, squeeze, shape = _as_2d(x)
    return _restore(gemm_f32(x2d, weight, transpose_b=True), squeeze, shape)


# ------------------------------------------------------------ quantizers

def _require_2d(name: str, weight: torch.Tensor) -> None:
    if weight.ndim != 2:
        raise ValueError(f"{name} must be 2D, got shape={tuple(weight.shape)}")


def _div32(a: torch.Tensor, b) -> torch.Tensor:
    """The correctly rounded fp32 quotient, as torch's CPU division gives it,
    on any device: the quotient of the fp32 operands in fp64, rounded once to
    fp32 (fp64 carries more than 2 x 24 + 2 bits, so rounding twice equals
    rounding once).  torch on the GPU divides by a Python scalar through its
    reciprocal, which rounds differently."""
    b = b.to(torch.float64) if isinstance(b, torch.Tensor) else float(b)
    return (a.to(torch.float64) / b).to(torch.float32)


def quantize_weight_i8_per_row(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """ckernel.py:70-75: scale = max|w|/127 (>= 1e-8), round half-even, clamp +-127."""
    if weight.dtype != torch.float32:
        raise ValueError(f"weight must be torch.float32, got {weight.dtype}")
    _require_2d("weight", weight)
    weight = weight.contiguous()
    max_abs = weight.abs().amax(dim=1)
    scales = torch.clamp(_div32(max_abs, 127.0), min=1e-8).to(torch.float32)
    qweight = torch.round(_div32(weight, scales.unsqueeze(1))).clamp(-127, 127).to(torch.int8).contiguous()
    return qweight, scales.contiguous()


def quantize_weight_i8_per_row_chunked(weight: torch.Tensor, rows_per_chunk: int = 1024):
    """ckernel.py:78-95, chunked over rows (outputs identical to the one-shot form)."""
    _require_2d("weight", weight)
    rows, cols = weight.shape
    rows_per_chunk = max(1, int(rows_per_chunk))
    qweight = torch.empty((rows, cols), dtype=torch.int8, device=weight.device)
    scales = torch.empty((rows,), dtype=torch.float32, device=weight.device)
    for start in range(0, rows, rows_per_chunk):
        end = min(start + rows_per_chunk, rows)
        q, s = quantize_weight_i8_per_row(weight[start:end].to(torch.float32))
        qweight[start:end].copy_(q)
        scales[start:end].copy_(s)
    return qweight.contiguous(), scales.contiguous()


def _pack_nibbles(q: torch.Tensor) -> torch.Tensor:
    if q.shape[1] % 2:
        q = torch.nn.functional.pad(q, (0, 1))
    low = torch.bitwise_and(q[:, 0::2], 0x0F).to(torch.uint8)
    high = torch.bitwise_left_shift(torch.bitwise_and(q[:, 1::2], 0x0F), 4).to(torch.uint8)
    return torch.bitwise_or(low, high)


def quantize_weight_i4_per_row_chunked(weight: torch.Tensor, rows_per_chunk: int = 1024):
    """ckernel.py:98-121: packed int4 [N, ceil(K/2)] (low nibble = even k), fp32 scales [N]."""
    _require_2d("weight", weight)
    rows, cols = weight.shape
    packed_cols = (cols + 1) // 2
    rows_per_chunk = max(1, int(rows_per_chunk))
    qweight = torch.empty((rows, packed_cols), dtype=torch.uint8, device=weight.device)
    scales = torch.empty((rows,), dtype=torch.float32, device=weight.device)
    for start in range(0, rows, rows_per_chunk):
        end = min(start + rows_per_chunk, rows)
        chunk = weight[start:end].to(torch.float32).contiguous()
        max_abs = chunk.abs().amax(dim=1)
        chunk_scales = torch.clamp(_div32(max_abs, 7.0), min=1e-8).to(torch.float32)
        q = torch.round(_div32(chunk, chunk_scales.unsqueeze(1))).clamp(-7, 7).to(torch.int16)
        qweight[start:end].copy_(_pack_nibbles(q))
        scales[start:end].copy_(chunk_scales)
    return qweight.contiguous(), scales.contiguous()


def quantize_weight_i4_grouped_chunked(weight: torch.Tensor, group_size: int = 32, rows_per_chunk: int = 1024):
    """ckernel.py:124-161: packed int4 with fp32 scales [N, ceil(K/G)]; the last
    partial group is zero-padded before its max is taken."""
    if group_size not in {32, 128}:
        raise ValueError("only group_size=32 or 128 is currently supported by the C kernel")
    _require_2d("weight", weight)
    rows, cols = weight.shape
    packed_cols = (cols + 1) // 2
    groups = (cols + group_size - 1) // group_size
    rows_per_chunk = max(1, int(rows_per_chunk))
    qweight = torch.empty((rows, packed_cols), dtype=torch.uint8, device=weight.device)
    scales = torch.empty((rows, groups), dtype=torch.float32, device=weight.device)
    for start in range(0, rows, rows_per_chunk):
        end = min(start + rows_per_chunk, rows)
        chunk = weight[start:end].to(torch.float32).contiguous()
        if cols % group_size:
            chunk = torch.nn.functional.pad(chunk, (0, groups * group_size - cols))
        grouped = chunk.reshape(end - start, groups, group_size)
        max_abs = grouped.abs().amax(dim=2)
        chunk_scales = torch.clamp(_div32(max_abs, 7.0), min=1e-8).to(torch.float32)
        q = torch.round(_div32(grouped, chunk_scales.unsqueeze(2))).clamp(-7, 7).to(torch.int16)
        q = q.reshape(end - start, groups * group_size)[:, :cols]
        qweight[start:end].copy_(_pack_nibbles(q))
        scales[start:end].copy_(chunk_scales)
    return qweight.contiguous(), scales.contiguous()


def unpack_i4_rows_to_i8(qweight: torch.Tensor, in_features: int | None = None) -> torch.Tensor:
    """ckernel.py:279-296: sign-extend each nibble (v >= 8 -> v - 16)."""
    if qweight.dtype != torch.uint8 or qweight.ndim != 2:
        raise ValueError("qweight must be a 2D torch.uint8 tensor")
    qweight = qweight.contiguous()
    n, packed_k = qweight.shape
    k = packed_k * 2 if in_features is None else int(in_features)
    if k <= 0 or packed_k != (k + 1) // 2:
        raise ValueError(f"incompatible W4 packed shape: qweight={tuple(qweight.shape)} in_features={in_features}")
    low = torch.bitwise_and(qweight, 0x0F).to(torch.int16)
    high = torch.bitwise_and(torch.bitwise_right_shift(qweight, 4), 0x0F).to(torch.int16)
    low = torch.where(low >= 8, low - 16, low)
    high = torch.where(high >= 8, high - 16, high)
    unpacked = torch.empty((n, packed_k * 2), dtype=torch.int8, device=qweight.device)
    unpacked[:, 0::2].copy_(low.to(torch.int8))
    unpacked[:, 1::2].copy_(high.to(torch.int8))
    return unpacked[:, :k].contiguous()


# --------------------------------------------------------------- linears

def _check_w8(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor, xdtype: torch.dtype, tag: str):
    if x.device.type != _GPU or x.dtype != xdtype or x.ndim != 2:
        raise ValueError(f"x must be a 2D GPU {xdtype} tensor")
    if qweight.device.type != _GPU or qweight.dtype != torch.int8 or qweight.ndim != 2:
        raise ValueError("qweight must be a 2D GPU torch.int8 tensor")
    if scales.device.type != _GPU or scales.dtype != torch.float32 or scales.ndim != 1:
        raise ValueError("scales must be a 1D GPU torch.float32 tensor")
    _same_device(x, qweight, scales)
    x, qweight, scales = x.contiguous(), qweight.contiguous(), scales.contiguous()
    m, k = x.shape
    n, wk = qweight.shape
    if wk != k or scales.shape[0] != n:
        raise ValueError(f"incompatible {tag} shapes: x={tuple(x.shape)} qweight={tuple(qweight.shape)} "
                         f"scales={tuple(scales.shape)}")
    return x, qweight, scales, m, n, k


def linear_w8a32(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """ckernel.py:164-180: fp32 x [M,K], int8 qweight [N,K], fp32 scales [N] -> fp32 [M,N]."""
    x, qweight, scales, m, n, k = _check_w8(x, qweight, scales, torch.float32, "W8A32")
    out = torch.empty((m, n), dtype=torch.float32, device=x.device)
    _bind_stream(x)
    rc = abi.linear_w8a32_ptr(x.data_ptr(), qweight.data_ptr(), scales.data_ptr(), out.data_ptr(), m, n, k)
    if rc != 0:
        raise _rc_error("ekernel_linear_w8a32", rc)
    return out


def linear_w8a16_bf16(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """ckernel.py:183-201: bf16 x, int8 qweight, fp32 scales -> bf16 [M,N]."""
    x, qweight, scales, m, n, k = _check_w8(x, qweight, scales, torch.bfloat16, "W8A16")
    out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    _bind_stream(x)
    rc = abi.linear_w8a16_bf16_ptr(x.data_ptr(), qweight.data_ptr(), scales.data_ptr(), out.data_ptr(), m, n, k)
    if rc != 0:
        raise _rc_error("ekernel_linear_w8a16_bf16", rc)
    return out


def linear_w8a16_bf16_argmax(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor) -> int:
    """ckernel.py:233-263: index of the largest bf16 logit of one row (ties ->
    lowest index); waits for the result."""
    x2d = _argmax_row(x)
    x2d, qweight, scales, m, n, k = _check_w8(x2d, qweight, scales, torch.bfloat16, "W8A16 argmax")
    _bind_stream(x2d)
    rc, index, _value = abi.linear_w8a16_bf16_argmax_ptr(x2d.data_ptr(), qweight.data_ptr(), scales.data_ptr(),
                                                         m, n, k)
    if rc != 0:
        raise _rc_error("ekernel_linear_w8a16_bf16_argmax", rc)
    return index


def linear_w8a16_bf16_argmax_device(x: torch.Tensor, qweight: torch.Tensor,
                                    scales: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """As linear_w8a16_bf16_argmax with the (index, value) left on the GPU --
    int64 [1] and float32 [1] tensors -- and no wait (usable under graph
    capture)."""
    x2d = _argmax_row(x)
    x2d, qweight, scales, m, n, k = _check_w8(x2d, qweight, scales, torch.bfloat16, "W8A16 argmax")
    index = torch.empty((1,), dtype=torch.int64, device=x2d.device)
    value = torch.empty((1,), dtype=torch.float32, device=x2d.device)
    _bind_stream(x2d)
    rc = abi.linear_w8a16_bf16_argmax_device_ptr(x2d.data_ptr(), qweight.data_ptr(), scales.data_ptr(),
                                                 index.data_ptr(), value.data_ptr(), m, n, k)
    if rc != 0:
        raise _rc_error("ekernel_linear_w8a16_bf16_argmax", rc)
    return index, value


def _argmax_row(x: torch.Tensor) -> torch.Tensor:
    if x.device.type != _GPU or x.dtype != torch.bfloat16:
        raise ValueError("x must be a GPU torch.bfloat16 tensor")
    if x.ndim == 1:
        return x.reshape(1, -1)
    if x.ndim == 2 and x.shape[0] == 1:
        return x
    raise ValueError(f"x must be a single row, got shape={tuple(x.shape)}")


def _check_w4(x, qweight, scales, in_features, scale_ndim: int):
    if x.device.type != _GPU or x.dtype != torch.bfloat16 or x.ndim != 2:
        raise ValueError("x must be a 2D GPU torch.bfloat16 tensor")
    if qweight.device.type != _GPU or qweight.dtype != torch.uint8 or qweight.ndim != 2:
        raise ValueError("qweight must be a 2D GPU torch.uint8 tensor")
    if scales.device.type != _GPU or scales.dtype != torch.float32 or scales.ndim != scale_ndim:
        raise ValueError(f"scales must be a {scale_ndim}D GPU torch.float32 tensor")
    _same_device(x, qweight, scales)
    x, qweight, scales = x.contiguous(), qweight.contiguous(), scales.contiguous()
    m, k = x.shape
    n, packed_k = qweight.shape
    if in_features is not None and int(in_features) != k:
        raise ValueError(f"in_features={in_features} does not match x K={k}")
    return x, qweight, scales, m, n, k, packed_k


def linear_w4a16_bf16(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
                      in_features: int | None = None) -> torch.Tensor:
    """ckernel.py:465-486: packed int4 with per-row fp32 scales [N]."""
    x, qweight, scales, m, n, k, packed_k = _check_w4(x, qweight, scales, in_features, 1)
    if packed_k != (k + 1) // 2 or scales.shape[0] != n:
        raise ValueError(f"incompatible W4A16 shapes: x={tuple(x.shape)} qweight={tuple(qweight.shape)} "
                         f"scales={tuple(scales.shape)}")
    out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    _bind_stream(x)
    rc = abi.linear_w4a16_bf16_ptr(x.data_ptr(), qweight.data_ptr(), scales.data_ptr(), out.data_ptr(), m, n, k)
    if rc != 0:
        raise _rc_error("ekernel_linear_w4a16_bf16", rc)
    return out


def _linear_w4g(x, qweight, scales, in_features, group: int):
    x, qweight, scales, m, n, k, packed_k = _check_w4(x, qweight, scales, in_features, 2)
    groups = (k + group - 1) // group
    if packed_k != (k + 1) // 2 or tuple(scales.shape) != (n, groups):
        raise ValueError(f"incompatible W4A16G{group} shapes: x={tuple(x.shape)} qweight={tuple(qweight.shape)} "
                         f"scales={tuple(scales.shape)}")
    out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    _bind_stream(x)
    fn = abi.linear_w4a16g128_bf16_ptr if group == 128 else abi.linear_w4a16g32_bf16_ptr
    rc = fn(x.data_ptr(), qweight.data_ptr(), scales.data_ptr(), out.data_ptr(), m, n, k)
    if rc != 0:
        raise _rc_error(f"ekernel_linear_w4a16g{group}_bf16", rc)
    return out


def linear_w4a16g32_bf16(x, qweight, scales, in_features=None) -> torch.Tensor:
    """ckernel.py:521-542: packed int4 with fp32 scales [N, ceil(K/32)]."""
    return _linear_w4g(x, qweight, scales, in_features, 32)


def linear_w4a16g128_bf16(x, qweight, scales, in_features=None) -> torch.Tensor:
    """ckernel.py:545-566: packed int4 with fp32 scales [N, ceil(K/128)]."""
    return _linear_w4g(x, qweight, scales, in_features, 128)


def swiglu_bf16(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """ckernel.py:569-583: bf16(silu(gate) * up)."""
    if gate.device.type != _GPU or up.device.type != _GPU:
        raise ValueError("gate and up must be GPU tensors")
    if gate.dtype != torch.bfloat16 or up.dtype != torch.bfloat16:
        raise ValueError("gate and up must be torch.bfloat16")
    if tuple(gate.shape) != tuple(up.shape):
        raise ValueError(f"gate/up shapes differ: gate={tuple(gate.shape)} up={tuple(up.shape)}")
    _same_device(gate, up)
    gate, up = gate.contiguous(), up.contiguous()
    out = torch.empty_like(gate)
    _bind_stream(gate)
    rc = abi.swiglu_bf16_ptr(gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.numel())
    if rc != 0:
        raise _rc_error("ekernel_swiglu_bf16", rc)
    return out


def silu_mul_bf16(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """torch.nn.functional.silu(gate) * up on bf16 tensors with the roundings
    of torch's CPU kernels (silu rounded to bf16, then the product): the
    reference's default activation between gate/up and down (linear.py:408-421,
    534-545), on the device."""
    if gate.device.type != _GPU or up.device.type != _GPU:
        raise ValueError("gate and up must be GPU tensors")
    if gate.dtype != torch.bfloat16 or up.dtype != torch.bfloat16:
        raise ValueError("gate and up must be torch.bfloat16")
    if tuple(gate.shape) != tuple(up.shape):
        raise ValueError(f"gate/up shapes differ: gate={tuple(gate.shape)} up={tuple(up.shape)}")
    _same_device(gate, up)
    gate, up = gate.contiguous(), up.contiguous()
    out = torch.empty_like(gate)
    n = gate.shape[-1] if gate.ndim else 1
    rows = gate.numel() // max(n, 1)
    _bind_stream(gate)
    rc = abi._load_lib().ekernel_silu_mul_bf16(ctypes.c_void_p(gate.data_ptr()), ctypes.c_void_p(up.data_ptr()),
                                               rows, n, n, ctypes.c_void_p(out.data_ptr()))
    if rc != 0:
        raise _rc_error("ekernel_silu_mul_bf16", rc)
    return out


def swiglu_w4a16_bf16(
    x: torch.Tensor,
    gate_up_qweight: torch.Tensor,
    gate_up_scales: torch.Tensor,
    down_qweight: torch.Tensor,
    down_scales: torch.Tensor,
    intermediate_size: int,
    gate_up_in_features: int | None = None,
    down_in_features: int | None = None,
) -> torch.Tensor:
    """ckernel.py:585-649: the fused W4 SwiGLU MLP of one token (M = 1)."""
    if x.device.type != _GPU or x.dtype != torch.bfloat16 or x.ndim != 2:
        raise ValueError("x must be a 2D GPU torch.bfloat16 tensor")
    if gate_up_qweight.device.type != _GPU or gate_up_qweight.dtype != torch.uint8 or gate_up_qweight.ndim != 2:
        raise ValueError("gate_up_qweight must be a 2D GPU torch.uint8 tensor")
    if down_qweight.device.type != _GPU or down_qweight.dtype != torch.uint8 or down_qweight.ndim != 2:
        raise ValueError("down_qweight must be a 2D GPU torch.uint8 tensor")
    if gate_up_scales.device.type != _GPU or gate_up_scales.dtype != torch.float32 or gate_up_scales.ndim != 1:
        raise ValueError("gate_up_scales must be a 1D GPU torch.float32 tensor")
    if down_scales.device.type != _GPU or down_scales.dtype != torch.float32 or down_scales.ndim != 1:
        raise ValueError("down_scales must be a 1D GPU torch.float32 tensor")
    _same_device(x, gate_up_qweight, gate_up_scales, down_qweight, down_scales)
    x = x.contiguous()
    gate_up_qweight = gate_up_qweight.contiguous()
    gate_up_scales = gate_up_scales.contiguous()
    down_qweight = down_qweight.contiguous()
    down_scales = down_scales.contiguous()
    m, k = x.shape
    intermediate_size = int(intermediate_size)
    gate_up_in_features = k if gate_up_in_features is None else int(gate_up_in_features)
    down_in_features = intermediate_size if down_in_features is None else int(down_in_features)
    hidden_size = int(down_qweight.shape[0])
    if m != 1:
        raise ValueError("experimental fused W4 SwiGLU currently supports M=1 only")
    if gate_up_in_features != k:
        raise ValueError(f"gate_up_in_features={gate_up_in_features} does not match x K={k}")
    if down_in_features != intermediate_size:
        raise ValueError("down_in_features must equal intermediate_size")
    if tuple(gate_up_qweight.shape) != (intermediate_size * 2, (gate_up_in_features + 1) // 2):
        raise ValueError(
            "gate_up_qweight shape must be "
            f"{(intermediate_size * 2, (gate_up_in_features + 1) // 2)}, got {tuple(gate_up_qweight.shape)}")
    if down_qweight.shape[1] != (down_in_features + 1) // 2:
        raise ValueError(f"down_qweight packed K does not match down_in_features={down_in_features}")
    if gate_up_scales.shape[0] != intermediate_size * 2 or down_scales.shape[0] != hidden_size:
        raise ValueError("scale shapes do not match qweight rows")
    out = torch.empty((m, hidden_size), dtype=torch.bfloat16, device=x.device)
    _bind_stream(x)
    rc = abi.swiglu_w4a16_bf16_ptr(x.data_ptr(), gate_up_qweight.data_ptr(), gate_up_scales.data_ptr(),
                                   down_qweight.data_ptr(), down_scales.data_ptr(), out.data_ptr(), m,
                                   hidden_size, intermediate_size, gate_up_in_features, down_in_features)
    if rc != 0:
        raise _rc_error("ekernel_swiglu_w4a16_bf16", rc)
    return out
