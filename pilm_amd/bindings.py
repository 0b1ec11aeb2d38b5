"""ctypes bindings to the HIP libecpu (pilm_amd/lib/libecpu.so).

Mirrors src/abi/bindings.py of piLM: the same loader search
(`PILM_ECPU_LIB` first, bindings.py:28-57), the same required symbols and
argtypes (`_configure`, bindings.py:59-233), the same ctypes structures
(bindings.py:235-289) and the same `*_ptr` helpers returning the C rc
(bindings.py:352-505).  Pointers handed to the linear kernels are device
(HBM) pointers; the library rejects anything else with ECPU_ERR_PARAM.

There is no CPU fallback: if the library cannot be found or lacks a symbol,
loading raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

_lib = None
_lib_path = None

_REQUIRED_SYMBOLS = [
    "ecpu_version", "ecpu_last_error", "ecpu_config_default", "ecpu_init", "ecpu_is_initialized",
    "ecpu_shutdown", "ekernel_detect_isa", "ekernel_isa_name", "edevice_active", "ekernel_gemm",
    "ekernel_linear_w8a32", "ekernel_linear_w8a16_bf16", "ekernel_swiglu_bf16",
]

_OPTIONAL_KERNEL_SYMBOLS = [
    "ekernel_gemm",
    "ekernel_linear_w8a32",
    "ekernel_linear_w8a16_bf16",
    "ekernel_linear_w8a16_bf16_argmax",
    "ekernel_linear_w8a16_bf16_i8b8",
    "ekernel_linear_w8a16_bf16_q8",
    "ekernel_linear_w4a16_bf16",
    "ekernel_linear_w4a16g32_bf16",
    "ekernel_linear_w4a16g128_bf16",
    "ekernel_linear_w4a16_bf16_q8",
    "ekernel_linear_w4a16_bf16_i4b8",
    "ekernel_linear_w4a16_bf16_b8",
    "ekernel_swiglu_bf16",
    "ekernel_swiglu_w4a16_bf16",
    "ekernel_rmsnorm_bf16",
    "ekernel_gated_delta_recurrent_f32",
    "ekernel_paged_attention_bf16",
    "ekernel_rmsnorm_gemma_bf16",
    "ekernel_qk_norm_rope_bf16",
    "ekernel_attention_exact_bf16",
    "ekernel_decode_attention_bf16",
    "ekernel_rmsnorm_linear_w4a16g128_bf16",
    "ekernel_silu_mul_bf16",
    "ekernel_greedy_step_bf16",
    "ekernel_qk_norm_rope_batch_bf16",
    "ekernel_attention_exact_batch_bf16",
]

DEFAULT_LIB = Path(__file__).resolve().parent / "lib" / "libecpu.so"

ECPU_OK = 0
ECPU_ERR_PARAM = -1
ECPU_ERR_MEM = -2
ECPU_ERR_DEVICE = -3
ECPU_ERR_KERNEL = -4
ECPU_ERR_UNSUPPORTED = -5


def _load_lib():
    global _lib, _lib_path
    if _lib is not None:
        return _lib
    candidates = []
    env_lib = os.environ.get("PILM_ECPU_LIB")
    if env_lib:
        candidates.append(Path(env_lib))
    candidates.append(DEFAULT_LIB)
    for c in candidates:
        if c.exists():
            lib = ctypes.CDLL(str(c))
            _configure(lib)
            _lib = lib
            _lib_path = str(c)
            return _lib
    raise RuntimeError(
        f"HIP libecpu not found (looked in {[str(c) for c in candidates]}); "
        "build it with `python -m pilm_amd.build`")


class EcpuConfig(ctypes.Structure):
    _fields_ = [
        ("n_threads", ctypes.c_int),
        ("numa_policy", ctypes.c_int),
        ("disable_amx", ctypes.c_int),
        ("disable_avx512", ctypes.c_int),
        ("eram_budget_bytes", ctypes.c_size_t),
        ("kv_cache_budget_bytes", ctypes.c_size_t),
        ("device_type", ctypes.c_int),
    ]


class EdeviceVtable(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("id", ctypes.c_int),
        ("caps", ctypes.c_uint64),
        ("alloc", ctypes.c_void_p),
        ("free", ctypes.c_void_p),
        ("memcpy_h2d", ctypes.c_void_p),
        ("memcpy_d2h", ctypes.c_void_p),
        ("memcpy_d2d", ctypes.c_void_p),
        ("synchronize", ctypes.c_void_p),
        ("mem_total", ctypes.c_void_p),
        ("mem_free", ctypes.c_void_p),
        ("init", ctypes.c_void_p),
        ("shutdown", ctypes.c_void_p),
    ]


class EkernelGemmDesc(ctypes.Structure):
    _fields_ = [
        ("M", ctypes.c_size_t),
        ("N", ctypes.c_size_t),
        ("K", ctypes.c_size_t),
        ("a_prec", ctypes.c_int),
        ("b_prec", ctypes.c_int),
        ("out_prec", ctypes.c_int),
        ("transpose_a", ctypes.c_int),
        ("transpose_b", ctypes.c_int),
    ]


class EkernelLinearW8A32Desc(ctypes.Structure):
    _fields_ = [
        ("M", ctypes.c_size_t),
        ("N", ctypes.c_size_t),
        ("K", ctypes.c_size_t),
    ]


class EkernelW4A16SwiGLUDesc(ctypes.Structure):
    _fields_ = [
        ("M", ctypes.c_size_t),
        ("hidden_size", ctypes.c_size_t),
        ("intermediate_size", ctypes.c_size_t),
        ("gate_up_in_features", ctypes.c_size_t),
        ("down_in_features", ctypes.c_size_t),
    ]


class EkernelPagedAttentionDesc(ctypes.Structure):
    """ekernel_paged_attention_desc_t (no C counterpart: attention.py:95-139)."""
    _fields_ = [
        ("S", ctypes.c_size_t),
        ("n_heads", ctypes.c_size_t),
        ("n_kv_heads", ctypes.c_size_t),
        ("head_dim", ctypes.c_size_t),
        ("cache_len", ctypes.c_size_t),
        ("block_size", ctypes.c_size_t),
        ("num_blocks", ctypes.c_size_t),
        ("n_block_ids", ctypes.c_size_t),
        ("gate_stride", ctypes.c_size_t),
    ]


class EkernelRmsnormDesc(ctypes.Structure):
    """ekernel_rmsnorm_desc_t (no C counterpart: layers.py:130-147 runs in torch)."""
    _fields_ = [("rows", ctypes.c_size_t), ("hidden", ctypes.c_size_t), ("eps", ctypes.c_float)]


class EkernelNormLinearDesc(ctypes.Structure):
    """ekernel_norm_linear_desc_t (GemmaRMSNorm, layers.py:130-147, fused into
    the following W4A16 g128 Linear; with swiglu the SwiGLU product too)."""
    _fields_ = [("rows", ctypes.c_size_t), ("N", ctypes.c_size_t), ("K", ctypes.c_size_t),
                ("eps", ctypes.c_float), ("swiglu", ctypes.c_int)]


class EkernelQkRopeDesc(ctypes.Structure):
    """ekernel_qk_rope_desc_t (attention.py:82-97)."""
    _fields_ = [(n, ctypes.c_size_t) for n in ("S", "n_heads", "n_kv_heads", "head_dim", "rot_dim", "q_stride",
                                               "kv_stride", "pos0", "max_positions", "block_size", "num_blocks",
                                               "n_block_ids")] + [("eps", ctypes.c_float)]


class EkernelAttentionExactDesc(ctypes.Structure):
    """ekernel_attention_exact_desc_t (attention.py:99-139)."""
    _fields_ = [(n, ctypes.c_size_t) for n in ("S", "n_heads", "n_kv_heads", "head_dim", "cache_len", "block_size",
                                               "num_blocks", "n_block_ids", "gate_row_stride", "gate_head_stride")]


class EkernelBatchSeq(ctypes.Structure):
    """ekernel_batch_seq_t: one sequence's rows of a batched call."""
    _fields_ = [(n, ctypes.c_int32) for n in ("row0", "rows", "pos0", "table")]


_LINEAR_ARGTYPES = [ctypes.POINTER(EkernelLinearW8A32Desc), ctypes.c_void_p, ctypes.c_void_p,
                    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]


def _configure(lib):
    missing = [s for s in _REQUIRED_SYMBOLS if not hasattr(lib, s)]
    if missing:
        raise AttributeError(f"libecpu is missing required symbols: {missing}")
    lib.ecpu_version.restype = ctypes.c_char_p
    lib.ecpu_last_error.restype = ctypes.c_char_p
    lib.ecpu_config_default.restype = EcpuConfig
    lib.ecpu_init.argtypes = [ctypes.POINTER(EcpuConfig)]
    lib.ecpu_init.restype = ctypes.c_int
    lib.ecpu_is_initialized.restype = ctypes.c_int
    lib.ekernel_detect_isa.restype = ctypes.c_int
    lib.ekernel_isa_name.argtypes = [ctypes.c_int]
    lib.ekernel_isa_name.restype = ctypes.c_char_p
    lib.edevice_active.restype = ctypes.POINTER(EdeviceVtable)
    lib.ecpu_shutdown.argtypes = []
    lib.ecpu_shutdown.restype = None
    lib.ekernel_gemm.argtypes = [ctypes.POINTER(EkernelGemmDesc), ctypes.c_void_p, ctypes.c_void_p,
                                 ctypes.c_void_p, ctypes.c_int]
    lib.ekernel_gemm.restype = ctypes.c_int
    for name in ("ekernel_linear_w8a32", "ekernel_linear_w8a16_bf16", "ekernel_linear_w4a16_bf16",
                 "ekernel_linear_w4a16g32_bf16", "ekernel_linear_w4a16g128_bf16"):
        if hasattr(lib, name):
            fn = getattr(lib, name)
            fn.argtypes = _LINEAR_ARGTYPES
            fn.restype = ctypes.c_int
    lib.ekernel_swiglu_bf16.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    lib.ekernel_swiglu_bf16.restype = ctypes.c_int
    if hasattr(lib, "ekernel_linear_w8a16_bf16_argmax"):
        # out_index / out_value as plain pointers: host (ctypes byref) or device
        lib.ekernel_linear_w8a16_bf16_argmax.argtypes = [
            ctypes.POINTER(EkernelLinearW8A32Desc), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        lib.ekernel_linear_w8a16_bf16_argmax.restype = ctypes.c_int
    if hasattr(lib, "ekernel_linear_w8a16_bf16_argmax_noalloc"):
        lib.ekernel_linear_w8a16_bf16_argmax_noalloc.argtypes = lib.ekernel_linear_w8a16_bf16_argmax.argtypes
        lib.ekernel_linear_w8a16_bf16_argmax_noalloc.restype = ctypes.c_int
    if hasattr(lib, "ekernel_swiglu_w4a16_bf16"):
        lib.ekernel_swiglu_w4a16_bf16.argtypes = [
            ctypes.POINTER(EkernelW4A16SwiGLUDesc), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        lib.ekernel_swiglu_w4a16_bf16.restype = ctypes.c_int
    if hasattr(lib, "ecpu_hip_profile_read"):
        lib.ecpu_hip_profile_begin.restype = ctypes.c_int
        lib.ecpu_hip_profile_end.restype = ctypes.c_int
        lib.ecpu_hip_profile_read.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
        lib.ecpu_hip_profile_read.restype = ctypes.c_int
    if hasattr(lib, "eram_hip_load_file"):
        lib.eram_hip_load_file.argtypes = [ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t),
                                           ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_void_p)]
        lib.eram_hip_load_file.restype = ctypes.c_int
        lib.eram_buffer_alloc.argtypes = [ctypes.c_size_t, ctypes.c_int]
        lib.eram_buffer_alloc.restype = ctypes.c_void_p
        lib.eram_buffer_free.argtypes = [ctypes.c_void_p]
        lib.eram_buffer_free.restype = None
        lib.eram_buffer_data.argtypes = [ctypes.c_void_p]
        lib.eram_buffer_data.restype = ctypes.c_void_p
        lib.eram_buffer_size.argtypes = [ctypes.c_void_p]
        lib.eram_buffer_size.restype = ctypes.c_size_t
        lib.eram_mmap.argtypes = [ctypes.c_char_p, ctypes.c_int]
        lib.eram_mmap.restype = ctypes.c_void_p
        lib.eram_munmap.argtypes = [ctypes.c_void_p]
        lib.eram_munmap.restype = ctypes.c_int
    if hasattr(lib, "ekernel_paged_attention_bf16"):
        lib.ekernel_paged_attention_bf16.argtypes = [ctypes.POINTER(EkernelPagedAttentionDesc)] + \
            [ctypes.c_void_p] * 8
        lib.ekernel_paged_attention_bf16.restype = ctypes.c_int
    if hasattr(lib, "ekernel_rmsnorm_gemma_bf16"):
        lib.ekernel_rmsnorm_gemma_bf16.argtypes = [ctypes.POINTER(EkernelRmsnormDesc)] + [ctypes.c_void_p] * 5
        lib.ekernel_rmsnorm_gemma_bf16.restype = ctypes.c_int
        lib.ekernel_qk_norm_rope_bf16.argtypes = [ctypes.POINTER(EkernelQkRopeDesc)] + [ctypes.c_void_p] * 12
        lib.ekernel_qk_norm_rope_bf16.restype = ctypes.c_int
        lib.ekernel_attention_exact_bf16.argtypes = [ctypes.POINTER(EkernelAttentionExactDesc)] + \
            [ctypes.c_void_p] * 7
        lib.ekernel_attention_exact_bf16.restype = ctypes.c_int
        lib.ekernel_decode_attention_bf16.argtypes = [ctypes.POINTER(EkernelQkRopeDesc)] + [ctypes.c_void_p] * 12
        lib.ekernel_decode_attention_bf16.restype = ctypes.c_int
        lib.ekernel_rmsnorm_linear_w4a16g128_bf16.argtypes = [ctypes.POINTER(EkernelNormLinearDesc)] + \
            [ctypes.c_void_p] * 7
        lib.ekernel_rmsnorm_linear_w4a16g128_bf16.restype = ctypes.c_int
        lib.ekernel_qk_norm_rope_batch_bf16.argtypes = [ctypes.POINTER(EkernelQkRopeDesc),
                                                        ctypes.POINTER(EkernelBatchSeq), ctypes.c_size_t,
                                                        ctypes.c_size_t] + [ctypes.c_void_p] * 11
        lib.ekernel_qk_norm_rope_batch_bf16.restype = ctypes.c_int
        lib.ekernel_attention_exact_batch_bf16.argtypes = [ctypes.POINTER(EkernelAttentionExactDesc),
                                                           ctypes.POINTER(EkernelBatchSeq), ctypes.c_size_t,
                                                           ctypes.c_size_t] + [ctypes.c_void_p] * 6
        lib.ekernel_attention_exact_batch_bf16.restype = ctypes.c_int
        lib.ekernel_silu_mul_bf16.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t,
                                              ctypes.c_size_t, ctypes.c_void_p]
        lib.ekernel_silu_mul_bf16.restype = ctypes.c_int
        lib.ekernel_greedy_step_bf16.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                                 ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.ekernel_greedy_step_bf16.restype = ctypes.c_int
    if hasattr(lib, "ecpu_hip_set_matrix_core_min_rows"):
        lib.ecpu_hip_set_matrix_core_min_rows.argtypes = [ctypes.c_int]
        lib.ecpu_hip_set_matrix_core_min_rows.restype = ctypes.c_int
        lib.ecpu_hip_matrix_core_min_rows.argtypes = []
        lib.ecpu_hip_matrix_core_min_rows.restype = ctypes.c_int
    if hasattr(lib, "ecpu_hip_set_stream"):
        lib.ecpu_hip_set_stream.argtypes = [ctypes.c_void_p]
        lib.ecpu_hip_set_stream.restype = ctypes.c_int
        lib.ecpu_hip_get_stream.argtypes = []
        lib.ecpu_hip_get_stream.restype = ctypes.c_void_p


EDEV_ECPU = 0
EDEV_CUDA = 1
EDEV_HIP = 2

ECPU_PRECISION_F32 = 0
ECPU_PRECISION_F16 = 1
ECPU_PRECISION_BF16 = 2
ECPU_PRECISION_F8_E4M3 = 3
ECPU_PRECISION_F8_E5M2 = 4
ECPU_PRECISION_I8 = 5
ECPU_PRECISION_I4 = 6

ISA_NAMES = {0: "scalar", 1: "avx2", 2: "avx512", 3: "amx", 4: "neon", 5: "sve", 6: "gfx950"}


def library_info() -> dict:
    """What the loaded library is: its path, version string, the ISA it
    reports, and which of the optional entry points it exports."""
    lib = _load_lib()
    return {"path": _lib_path, "version": lib.ecpu_version().decode(),
            "isa": ISA_NAMES.get(lib.ekernel_detect_isa(), "unknown"),
            "entry_points": {name: hasattr(lib, name) for name in _OPTIONAL_KERNEL_SYMBOLS}}


def last_error() -> str | None:
    err = _load_lib().ecpu_last_error()
    return err.decode() if err else None


def shutdown():
    _load_lib().ecpu_shutdown()


def set_stream(stream_handle: int) -> None:
    """Make the library enqueue on this hipStream_t (0 = null stream)."""
    _load_lib().ecpu_hip_set_stream(ctypes.c_void_p(stream_handle or None))


def set_matrix_core_min_rows(rows: int) -> None:
    """Rows from which linears use the matrix cores (0 = never; < 0 = default)."""
    _load_lib().ecpu_hip_set_matrix_core_min_rows(int(rows))


def matrix_core_min_rows() -> int:
    return int(_load_lib().ecpu_hip_matrix_core_min_rows())


def profile_begin() -> None:
    """Start recording a HIP event pair around every linear call."""
    _load_lib().ecpu_hip_profile_begin()


def profile_end() -> None:
    _load_lib().ecpu_hip_profile_end()


def profile_read() -> dict:
    """{family: {"calls", "ms", "bytes", "flops"}} for the calls recorded so far."""
    lib = _load_lib()
    buf = ctypes.create_string_buffer(1 << 16)
    rc = lib.ecpu_hip_profile_read(buf, len(buf))
    if rc != 0:
        raise RuntimeError(f"ecpu_hip_profile_read failed: rc={rc} ({last_error()})")
    out = {}
    for line in buf.value.decode().splitlines():
        name, calls, ms, nbytes, flops = line.split()
        out[name] = {"calls": int(calls), "ms": float(ms), "bytes": float(nbytes), "flops": float(flops)}
    return out


def _linear_ptr(name: str, a_ptr: int, w_ptr: int, scales_ptr: int, c_ptr: int, m: int, n: int, k: int,
                isa: int | None) -> int:
    lib = _load_lib()
    if not hasattr(lib, name):
        raise RuntimeError(f"loaded eCPU library does not expose {name}")
    if isa is None:
        isa = lib.ekernel_detect_isa()
    desc = EkernelLinearW8A32Desc(m, n, k)
    return getattr(lib, name)(ctypes.byref(desc), ctypes.c_void_p(a_ptr), ctypes.c_void_p(w_ptr),
                              ctypes.c_void_p(scales_ptr), ctypes.c_void_p(c_ptr), int(isa))


def linear_w8a32_ptr(a_ptr, w_ptr, scales_ptr, c_ptr, m, n, k, isa=None) -> int:
    return _linear_ptr("ekernel_linear_w8a32", a_ptr, w_ptr, scales_ptr, c_ptr, m, n, k, isa)


def linear_w8a16_bf16_ptr(a_ptr, w_ptr, scales_ptr, c_ptr, m, n, k, isa=None) -> int:
    return _linear_ptr("ekernel_linear_w8a16_bf16", a_ptr, w_ptr, scales_ptr, c_ptr, m, n, k, isa)


def linear_w4a16_bf16_ptr(a_ptr, w_ptr, scales_ptr, c_ptr, m, n, k, isa=None) -> int:
    return _linear_ptr("ekernel_linear_w4a16_bf16", a_ptr, w_ptr, scales_ptr, c_ptr, m, n, k, isa)


def linear_w4a16g32_bf16_ptr(a_ptr, w_ptr, scales_ptr, c_ptr, m, n, k, isa=None) -> int:
    return _linear_ptr("ekernel_linear_w4a16g32_bf16", a_ptr, w_ptr, scales_ptr, c_ptr, m, n, k, isa)


def linear_w4a16g128_bf16_ptr(a_ptr, w_ptr, scales_ptr, c_ptr, m, n, k, isa=None) -> int:
    return _linear_ptr("ekernel_linear_w4a16g128_bf16", a_ptr, w_ptr, scales_ptr, c_ptr, m, n, k, isa)


def swiglu_bf16_ptr(gate_ptr: int, up_ptr: int, out_ptr: int, n: int) -> int:
    lib = _load_lib()
    return lib.ekernel_swiglu_bf16(ctypes.c_void_p(gate_ptr), ctypes.c_void_p(up_ptr),
                                   ctypes.c_void_p(out_ptr), ctypes.c_size_t(n))


def linear_w8a16_bf16_argmax_ptr(a_ptr: int, w_ptr: int, scales_ptr: int,
                                 m: int, n: int, k: int, isa: int | None = None) -> tuple[int, int, float]:
    """bindings.py:401-420: (rc, index, value), results returned through host memory."""
    lib = _load_lib()
    if not hasattr(lib, "ekernel_linear_w8a16_bf16_argmax"):
        raise RuntimeError("loaded eCPU library does not expose ekernel_linear_w8a16_bf16_argmax")
    if isa is None:
        isa = lib.ekernel_detect_isa()
    desc = EkernelLinearW8A32Desc(m, n, k)
    out_index = ctypes.c_size_t(0)
    out_value = ctypes.c_float(0.0)
    rc = lib.ekernel_linear_w8a16_bf16_argmax(
        ctypes.byref(desc), ctypes.c_void_p(a_ptr), ctypes.c_void_p(w_ptr), ctypes.c_void_p(scales_ptr),
        ctypes.addressof(out_index), ctypes.addressof(out_value), int(isa))
    return int(rc), int(out_index.value), float(out_value.value)


def linear_w8a16_bf16_argmax_device_ptr(a_ptr: int, w_ptr: int, scales_ptr: int, index_ptr: int, value_ptr: int,
                                        m: int, n: int, k: int, isa: int | None = None) -> int:
    """The same entry point with device outputs (size_t index, float value):
    enqueued on the current stream, no wait."""
    lib = _load_lib()
    if isa is None:
        isa = lib.ekernel_detect_isa()
    desc = EkernelLinearW8A32Desc(m, n, k)
    return lib.ekernel_linear_w8a16_bf16_argmax(
        ctypes.byref(desc), ctypes.c_void_p(a_ptr), ctypes.c_void_p(w_ptr), ctypes.c_void_p(scales_ptr),
        ctypes.c_void_p(index_ptr), ctypes.c_void_p(value_ptr), int(isa))


def swiglu_w4a16_bf16_ptr(x_ptr: int, gate_up_w_ptr: int, gate_up_scales_ptr: int,
                          down_w_ptr: int, down_scales_ptr: int, c_ptr: int,
                          m: int, hidden_size: int, intermediate_size: int,
                          gate_up_in_features: int, down_in_features: int,
                          isa: int | None = None) -> int:
    """bindings.py:567-593."""
    lib = _load_lib()
    if not hasattr(lib, "ekernel_swiglu_w4a16_bf16"):
        raise RuntimeError("loaded eCPU library does not expose ekernel_swiglu_w4a16_bf16")
    if isa is None:
        isa = lib.ekernel_detect_isa()
    desc = EkernelW4A16SwiGLUDesc(m, hidden_size, intermediate_size, gate_up_in_features, down_in_features)
    return lib.ekernel_swiglu_w4a16_bf16(
        ctypes.byref(desc), ctypes.c_void_p(x_ptr), ctypes.c_void_p(gate_up_w_ptr),
        ctypes.c_void_p(gate_up_scales_ptr), ctypes.c_void_p(down_w_ptr), ctypes.c_void_p(down_scales_ptr),
        ctypes.c_void_p(c_ptr), int(isa))


def paged_attention_bf16_ptr(q_ptr: int, k_new_ptr: int, v_new_ptr: int, k_cache_ptr: int, v_cache_ptr: int,
                             block_ids_ptr: int, gate_ptr: int, out_ptr: int, s: int, n_heads: int,
                             n_kv_heads: int, head_dim: int, cache_len: int, block_size: int, num_blocks: int,
                             n_block_ids: int, gate_stride: int) -> int:
    """Paged attention of one sequence (ekernel_paged_attention_bf16); 0 for
    k_cache_ptr / v_cache_ptr / gate_ptr means none.  Returns the C rc."""
    lib = _load_lib()
    if not hasattr(lib, "ekernel_paged_attention_bf16"):
        raise RuntimeError("loaded eCPU library does not expose ekernel_paged_attention_bf16")
    desc = EkernelPagedAttentionDesc(s, n_heads, n_kv_heads, head_dim, cache_len, block_size, num_blocks,
                                     n_block_ids, gate_stride)
    ptrs = [q_ptr, k_new_ptr, v_new_ptr, k_cache_ptr, v_cache_ptr, block_ids_ptr, gate_ptr, out_ptr]
    return lib.ekernel_paged_attention_bf16(ctypes.byref(desc), *[ctypes.c_void_p(p or None) for p in ptrs])


def eram_load_file(path: str, ranges) -> int:
    """Upload byte ranges of a file into device memory: ranges is a list of
    (file_offset, nbytes, device_ptr).  Returns the C rc; waits for the copies."""
    lib = _load_lib()
    n = len(ranges)
    offs = (ctypes.c_size_t * max(n, 1))(*[r[0] for r in ranges])
    sizes = (ctypes.c_size_t * max(n, 1))(*[r[1] for r in ranges])
    dsts = (ctypes.c_void_p * max(n, 1))(*[ctypes.c_void_p(r[2]) for r in ranges])
    return lib.eram_hip_load_file(str(path).encode(), n, offs, sizes, dsts)
