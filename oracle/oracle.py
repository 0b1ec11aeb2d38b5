"""Python face of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Loads oracle/_build/liboracle.so (the plain-C restatement in oracle.c) and,
when it has been built, oracle/_ref/libecpu_ref.so (the reference's own
kernels.c compiled from source by oracle/Makefile).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only to check or to time the CPU side.

The numpy functions below restate the reference's weight quantizers and the
W4 unpack helper (src/runtime/ckernel.py:70-161, 279-296).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "_build" / "liboracle.so"
REF_LIB = HERE / "_ref" / "libecpu_ref.so"

_P = ctypes.c_void_p
_S = ctypes.c_size_t


def build(ref: bool = True) -> None:
    """Compile the restatement (and the reference kernels when present)."""
    target = "all" if ref else "oracle"
    subprocess.run(["make", "-s", "-C", str(HERE), target], check=True)


class _Desc(ctypes.Structure):
    # ekernel_linear_w8a32_desc_t, src/ecpu/include/kernel/api.h:40-42
    _fields_ = [("M", _S), ("N", _S), ("K", _S)]


class _SwiGLUDesc(ctypes.Structure):
    # ekernel_w4a16_swiglu_desc_t, src/ecpu/include/kernel/api.h:44-50
    _fields_ = [("M", _S), ("hidden_size", _S), ("intermediate_size", _S), ("gate_up_in_features", _S),
                ("down_in_features", _S)]


_oracle = None
_ref = None
_planted: dict[int, ctypes.CDLL] = {}


def _configure_oracle(lib):
    lib.oracle_linear_w8a32.argtypes = [_S, _S, _S, _P, _P, _P, _P]
    lib.oracle_linear_w8a16_bf16.argtypes = [_S, _S, _S, _P, _P, _P, _P]
    lib.oracle_linear_w4a16_bf16.argtypes = [_S, _S, _S, _P, _P, _P, _P]
    lib.oracle_linear_w4a16g_bf16.argtypes = [_S, _S, _S, _S, _P, _P, _P, _P]
    lib.oracle_linear_w8a16_bf16_argmax.argtypes = [_S, _S, _P, _P, _P, ctypes.POINTER(_S),
                                                     ctypes.POINTER(ctypes.c_float)]
    lib.oracle_swiglu_bf16.argtypes = [_P, _P, _P, _S]
    lib.oracle_swiglu_w4a16_bf16.argtypes = [_S, _S, _S, _P, _P, _P, _P, _P, _P, _P]
    for f in ("oracle_linear_w8a32", "oracle_linear_w8a16_bf16", "oracle_linear_w4a16_bf16",
              "oracle_linear_w4a16g_bf16", "oracle_linear_w8a16_bf16_argmax", "oracle_swiglu_bf16",
              "oracle_swiglu_w4a16_bf16"):
        getattr(lib, f).restype = ctypes.c_int
    lib.oracle_expf.argtypes = [_P, _P, _S]
    lib.oracle_expf.restype = None
    return lib


def planted_lib(variant: int):
    """A deliberately wrong build of the restatement (ORACLE_PLANT=variant)."""
    if variant not in _planted:
        path = HERE / "_build" / f"liboracle_plant{variant}.so"
        # make rebuilds a variant older than oracle.c
        subprocess.run(["make", "-s", "-C", str(HERE), "plant", f"PLANT={variant}"], check=True)
        _planted[variant] = _configure_oracle(ctypes.CDLL(str(path)))
    return _planted[variant]


def oracle_lib():
    global _oracle
    if _oracle is None:
        if not ORACLE_LIB.exists() or (HERE / "oracle.c").stat().st_mtime > ORACLE_LIB.stat().st_mtime:
            build(ref=False)
        _oracle = _configure_oracle(ctypes.CDLL(str(ORACLE_LIB)))
    return _oracle


def ref_available() -> bool:
    return REF_LIB.exists()


def ref_lib():
    """The reference's kernels.c built from source; raises if not built."""
    global _ref
    if _ref is None:
        if not REF_LIB.exists():
            raise FileNotFoundError(f"{REF_LIB} not built (needs the reference sources)")
        lib = ctypes.CDLL(str(REF_LIB))
        for f in ("ekernel_linear_w8a32", "ekernel_linear_w8a16_bf16", "ekernel_linear_w4a16_bf16",
                  "ekernel_linear_w4a16g32_bf16", "ekernel_linear_w4a16g128_bf16"):
            getattr(lib, f).argtypes = [ctypes.POINTER(_Desc), _P, _P, _P, _P, ctypes.c_int]
            getattr(lib, f).restype = ctypes.c_int
        lib.ekernel_linear_w8a16_bf16_argmax.argtypes = [ctypes.POINTER(_Desc), _P, _P, _P,
                                                         ctypes.POINTER(_S), ctypes.POINTER(ctypes.c_float),
                                                         ctypes.c_int]
        lib.ekernel_linear_w8a16_bf16_argmax.restype = ctypes.c_int
        lib.ekernel_swiglu_bf16.argtypes = [_P, _P, _P, _S]
        lib.ekernel_swiglu_bf16.restype = ctypes.c_int
        lib.ekernel_swiglu_w4a16_bf16.argtypes = [ctypes.POINTER(_SwiGLUDesc), _P, _P, _P, _P, _P, _P, ctypes.c_int]
        lib.ekernel_swiglu_w4a16_bf16.restype = ctypes.c_int
        _ref = lib
    return _ref


def _olib(impl):
    """impl: "oracle" for the restatement, or an int for a planted variant."""
    return oracle_lib() if impl == "oracle" else planted_lib(int(impl))


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _check(rc: int, name: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{name} failed: rc={rc}")


# ---------------------------------------------------------------- linears

def linear_w8a32(x: np.ndarray, qweight: np.ndarray, scales: np.ndarray, impl: str = "oracle") -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    qweight = np.ascontiguousarray(qweight, np.int8)
    scales = np.ascontiguousarray(scales, np.float32)
    m, k = x.shape
    n = qweight.shape[0]
    out = np.empty((m, n), np.float32)
    if impl != "ref":
        rc = _olib(impl).oracle_linear_w8a32(m, n, k, _ptr(x), _ptr(qweight), _ptr(scales), _ptr(out))
    else:
        d = _Desc(m, n, k)
        rc = ref_lib().ekernel_linear_w8a32(ctypes.byref(d), _ptr(x), _ptr(qweight), _ptr(scales), _ptr(out), 1)
    _check(rc, "linear_w8a32")
    return out


def linear_w8a16_bf16(x_bits: np.ndarray, qweight: np.ndarray, scales: np.ndarray, impl: str = "oracle") -> np.ndarray:
    x_bits = np.ascontiguousarray(x_bits, np.uint16)
    qweight = np.ascontiguousarray(qweight, np.int8)
    scales = np.ascontiguousarray(scales, np.float32)
    m, k = x_bits.shape
    n = qweight.shape[0]
    out = np.empty((m, n), np.uint16)
    if impl != "ref":
        rc = _olib(impl).oracle_linear_w8a16_bf16(m, n, k, _ptr(x_bits), _ptr(qweight), _ptr(scales), _ptr(out))
    else:
        d = _Desc(m, n, k)
        rc = ref_lib().ekernel_linear_w8a16_bf16(ctypes.byref(d), _ptr(x_bits), _ptr(qweight), _ptr(scales),
                                                 _ptr(out), 1)
    _check(rc, "linear_w8a16_bf16")
    return out


def linear_w8a16_bf16_argmax(x_bits: np.ndarray, qweight: np.ndarray, scales: np.ndarray,
                             impl: str = "oracle") -> tuple[int, float]:
    x_bits = np.ascontiguousarray(x_bits, np.uint16).reshape(1, -1)
    qweight = np.ascontiguousarray(qweight, np.int8)
    scales = np.ascontiguousarray(scales, np.float32)
    k = x_bits.shape[1]
    n = qweight.shape[0]
    idx = _S(0)
    val = ctypes.c_float(0)
    if impl != "ref":
        rc = _olib(impl).oracle_linear_w8a16_bf16_argmax(n, k, _ptr(x_bits), _ptr(qweight), _ptr(scales),
                                                          ctypes.byref(idx), ctypes.byref(val))
    else:
        d = _Desc(1, n, k)
        rc = ref_lib().ekernel_linear_w8a16_bf16_argmax(ctypes.byref(d), _ptr(x_bits), _ptr(qweight),
                                                        _ptr(scales), ctypes.byref(idx), ctypes.byref(val), 1)
    _check(rc, "linear_w8a16_bf16_argmax")
    return int(idx.value), float(val.value)


def linear_w4a16_bf16(x_bits: np.ndarray, qweight: np.ndarray, scales: np.ndarray, impl: str = "oracle") -> np.ndarray:
    x_bits = np.ascontiguousarray(x_bits, np.uint16)
    qweight = np.ascontiguousarray(qweight, np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    m, k = x_bits.shape
    n = qweight.shape[0]
    out = np.empty((m, n), np.uint16)
    if impl != "ref":
        rc = _olib(impl).oracle_linear_w4a16_bf16(m, n, k, _ptr(x_bits), _ptr(qweight), _ptr(scales), _ptr(out))
    else:
        d = _Desc(m, n, k)
        rc = ref_lib().ekernel_linear_w4a16_bf16(ctypes.byref(d), _ptr(x_bits), _ptr(qweight), _ptr(scales),
                                                 _ptr(out), 1)
    _check(rc, "linear_w4a16_bf16")
    return out


def linear_w4a16g_bf16(x_bits: np.ndarray, qweight: np.ndarray, scales: np.ndarray, group_size: int,
                       impl: str = "oracle") -> np.ndarray:
    x_bits = np.ascontiguousarray(x_bits, np.uint16)
    qweight = np.ascontiguousarray(qweight, np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    m, k = x_bits.shape
    n = qweight.shape[0]
    out = np.empty((m, n), np.uint16)
    if impl != "ref":
        rc = _olib(impl).oracle_linear_w4a16g_bf16(m, n, k, group_size, _ptr(x_bits), _ptr(qweight),
                                                    _ptr(scales), _ptr(out))
    else:
        d = _Desc(m, n, k)
        fn = {32: ref_lib().ekernel_linear_w4a16g32_bf16, 128: ref_lib().ekernel_linear_w4a16g128_bf16}[group_size]
        rc = fn(ctypes.byref(d), _ptr(x_bits), _ptr(qweight), _ptr(scales), _ptr(out), 1)
    _check(rc, f"linear_w4a16g{group_size}_bf16")
    return out


# ------------------------------------------------------------- SwiGLU

def swiglu_bf16(g_bits: np.ndarray, u_bits: np.ndarray, impl: str = "oracle") -> np.ndarray:
    """kernels.c:1580-1596 on bf16 bit patterns of equal shape."""
    g_bits = np.ascontiguousarray(g_bits, np.uint16)
    u_bits = np.ascontiguousarray(u_bits, np.uint16)
    assert g_bits.shape == u_bits.shape
    out = np.empty_like(g_bits)
    if impl != "ref":
        rc = _olib(impl).oracle_swiglu_bf16(_ptr(g_bits), _ptr(u_bits), _ptr(out), g_bits.size)
    else:
        rc = ref_lib().ekernel_swiglu_bf16(_ptr(g_bits), _ptr(u_bits), _ptr(out), g_bits.size)
    _check(rc, "swiglu_bf16")
    return out


def swiglu_w4a16_bf16(x_bits: np.ndarray, gate_up_qweight: np.ndarray, gate_up_scales: np.ndarray,
                      down_qweight: np.ndarray, down_scales: np.ndarray, intermediate_size: int,
                      impl: str = "oracle", return_hidden: bool = False):
    """kernels.c:1598-1735: x [1, K] bf16, gate_up int4 [2I, ceil(K/2)] with
    scales [2I], down int4 [H, ceil(I/2)] with scales [H] -> bf16 [1, H]
    (and, for the restatement, the bf16 hidden row [I])."""
    x_bits = np.ascontiguousarray(x_bits, np.uint16).reshape(1, -1)
    gu = np.ascontiguousarray(gate_up_qweight, np.uint8)
    gs = np.ascontiguousarray(gate_up_scales, np.float32)
    dw = np.ascontiguousarray(down_qweight, np.uint8)
    ds = np.ascontiguousarray(down_scales, np.float32)
    k = x_bits.shape[1]
    i_sz = int(intermediate_size)
    h = dw.shape[0]
    assert gu.shape == (2 * i_sz, (k + 1) // 2) and gs.shape == (2 * i_sz,)
    assert dw.shape == (h, (i_sz + 1) // 2) and ds.shape == (h,)
    out = np.empty((1, h), np.uint16)
    hidden = np.empty((i_sz,), np.uint16)
    if impl != "ref":
        rc = _olib(impl).oracle_swiglu_w4a16_bf16(h, i_sz, k, _ptr(x_bits), _ptr(gu), _ptr(gs), _ptr(dw), _ptr(ds),
                                                  _ptr(out), _ptr(hidden))
    else:
        d = _SwiGLUDesc(1, h, i_sz, k, i_sz)
        rc = ref_lib().ekernel_swiglu_w4a16_bf16(ctypes.byref(d), _ptr(x_bits), _ptr(gu), _ptr(gs), _ptr(dw),
                                                 _ptr(ds), _ptr(out), 1)
    _check(rc, "swiglu_w4a16_bf16")
    return (out, hidden) if return_hidden and impl != "ref" else out


def expf(x: np.ndarray) -> np.ndarray:
    """The C library's expf, element by element."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    oracle_lib().oracle_expf(_ptr(x), _ptr(out), x.size)
    return out


# ------------------------------------------------- quantizers (ckernel.py)

def quantize_weight_i8_per_row(weight: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """src/runtime/ckernel.py:70-95: scale = max|w|/127 (>= 1e-8), RNE, clamp +-127."""
    w = np.ascontiguousarray(weight, np.float32)
    scales = np.maximum(np.abs(w).max(axis=1) / np.float32(127.0), np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.round(w / scales[:, None]), -127, 127).astype(np.int8)
    return q, scales


def _pack_nibbles(q: np.ndarray) -> np.ndarray:
    rows, cols = q.shape
    if cols % 2:
        q = np.pad(q, ((0, 0), (0, 1)))
    low = (q[:, 0::2] & 0x0F).astype(np.uint8)
    high = ((q[:, 1::2] & 0x0F) << 4).astype(np.uint8)
    return (low | high).astype(np.uint8)


def quantize_weight_i4_per_row(weight: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """src/runtime/ckernel.py:98-121: scale = max|w|/7 (>= 1e-8), RNE, clamp +-7, pack."""
    w = np.ascontiguousarray(weight, np.float32)
    scales = np.maximum(np.abs(w).max(axis=1) / np.float32(7.0), np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.round(w / scales[:, None]), -7, 7).astype(np.int16)
    return _pack_nibbles(q), scales


def quantize_weight_i4_grouped(weight: np.ndarray, group_size: int) -> tuple[np.ndarray, np.ndarray]:
    """src/runtime/ckernel.py:124-161: per-group scales over zero-padded groups."""
    if group_size not in (32, 128):
        raise ValueError("only group_size=32 or 128 is currently supported by the C kernel")
    w = np.ascontiguousarray(weight, np.float32)
    rows, cols = w.shape
    groups = (cols + group_size - 1) // group_size
    padded = np.pad(w, ((0, 0), (0, groups * group_size - cols)))
    g = padded.reshape(rows, groups, group_size)
    scales = np.maximum(np.abs(g).max(axis=2) / np.float32(7.0), np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.round(g / scales[:, :, None]), -7, 7).astype(np.int16)
    q = q.reshape(rows, groups * group_size)[:, :cols]
    return _pack_nibbles(q), scales


def unpack_i4_rows_to_i8(qweight: np.ndarray, in_features: int | None = None) -> np.ndarray:
    """src/runtime/ckernel.py:279-296 (and kernels.c:43-46): sign-extend nibbles."""
    q = np.ascontiguousarray(qweight, np.uint8)
    n, pk = q.shape
    k = pk * 2 if in_features is None else int(in_features)
    if k <= 0 or pk != (k + 1) // 2:
        raise ValueError(f"incompatible W4 packed shape: qweight={q.shape} in_features={in_features}")
    low = (q & 0x0F).astype(np.int16)
    high = (q >> 4).astype(np.int16)
    low = np.where(low >= 8, low - 16, low)
    high = np.where(high >= 8, high - 16, high)
    out = np.empty((n, pk * 2), np.int8)
    out[:, 0::2] = low
    out[:, 1::2] = high
    return np.ascontiguousarray(out[:, :k])


def dequantize_w4(qweight: np.ndarray, scales: np.ndarray, in_features: int) -> np.ndarray:
    """w[n,k] = sext4(nibble) * scale[n, k // G] in fp32 (G = K for per-row scales)."""
    q = unpack_i4_rows_to_i8(qweight, in_features).astype(np.float32)
    if scales.ndim == 1:
        return q * scales[:, None]
    groups = scales.shape[1]
    gsize = 128 if groups == (in_features + 127) // 128 else 32
    idx = np.arange(in_features) // gsize
    return q * scales[:, idx]
