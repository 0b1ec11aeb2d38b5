"""The C-ABI library loads and exports every symbol include/ecpu_hip.h declares
(no GPU needed: nothing here launches a kernel)."""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from pilm_amd import bindings as abi

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "ecpu_hip.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"typedef struct edevice_vtable \{.*?\} edevice_vtable_t;", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w\s\*]*?\b(\w+)\s*\([^;{]*\)\s*;", text, flags=re.M)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib_path() -> Path:
    p = abi.DEFAULT_LIB
    if not p.exists():
        pytest.fail(f"{p} is not built; run python -m pilm_amd.build")
    return p


def test_header_declares_the_reference_abi():
    names = declared_functions()
    for required in abi._REQUIRED_SYMBOLS:
        if required.startswith(("ecpu_", "ekernel_", "edevice_")):
            assert required in names, required
    for hot in ("ekernel_linear_w4a16_bf16", "ekernel_linear_w4a16g32_bf16", "ekernel_linear_w4a16g128_bf16"):
        assert hot in names


def test_every_declared_symbol_is_exported(lib_path):
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib_path)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing


def test_library_loads_and_configures(lib_path):
    lib = abi._load_lib()
    info = abi.library_info()
    assert info["path"] == str(lib_path)
    assert info["version"].endswith("gfx950")
    assert info["isa"] == "gfx950"
    assert all(info["entry_points"][s] for s in (
        "ekernel_gemm", "ekernel_linear_w8a32", "ekernel_linear_w8a16_bf16", "ekernel_linear_w4a16_bf16",
        "ekernel_linear_w4a16g32_bf16", "ekernel_linear_w4a16g128_bf16", "ekernel_swiglu_bf16",
        "ekernel_linear_w8a16_bf16_argmax", "ekernel_swiglu_w4a16_bf16", "ekernel_rmsnorm_gemma_bf16",
        "ekernel_qk_norm_rope_bf16", "ekernel_attention_exact_bf16", "ekernel_silu_mul_bf16",
        "ekernel_greedy_step_bf16", "ekernel_qk_norm_rope_batch_bf16", "ekernel_attention_exact_batch_bf16"))
    vt = lib.edevice_get  # exported registry accessor
    assert vt is not None


def test_descriptor_layout_matches_reference():
    # ekernel_linear_w8a32_desc_t (kernel/api.h:40-42) and ecpu_config_t (ecpu.h:23-31)
    assert ctypes.sizeof(abi.EkernelLinearW8A32Desc) == 24
    assert abi.EcpuConfig.device_type.offset == 32
    assert ctypes.sizeof(abi.EkernelGemmDesc) == 44 or ctypes.sizeof(abi.EkernelGemmDesc) == 48
    # ekernel_w4a16_swiglu_desc_t (kernel/api.h:44-50): five size_t
    assert ctypes.sizeof(abi.EkernelW4A16SwiGLUDesc) == 40
    assert abi.EkernelW4A16SwiGLUDesc.down_in_features.offset == 32
    # the decoder steps' descriptors (ecpu_hip.h): size_t fields, then the float eps
    assert abi.EkernelRmsnormDesc.eps.offset == 16 and ctypes.sizeof(abi.EkernelRmsnormDesc) == 24
    assert abi.EkernelQkRopeDesc.eps.offset == 96 and ctypes.sizeof(abi.EkernelQkRopeDesc) == 104
    assert ctypes.sizeof(abi.EkernelAttentionExactDesc) == 80
    assert abi.EkernelNormLinearDesc.eps.offset == 24 and abi.EkernelNormLinearDesc.swiglu.offset == 28
    assert ctypes.sizeof(abi.EkernelNormLinearDesc) == 32
    # ekernel_batch_seq_t: four int32
    assert ctypes.sizeof(abi.EkernelBatchSeq) == 16 and abi.EkernelBatchSeq.table.offset == 12


def test_missing_symbol_fails_loudly(tmp_path, monkeypatch):
    """A library without the required symbols is refused, as bindings.py:_configure does."""
    src = tmp_path / "empty.c"
    src.write_text("int unrelated(void) { return 0; }\n")
    so = tmp_path / "libempty.so"
    subprocess.run(["gcc", "-shared", "-fPIC", "-o", str(so), str(src)], check=True)
    monkeypatch.setattr(abi, "_lib", None)
    monkeypatch.setenv("PILM_ECPU_LIB", str(so))
    with pytest.raises(AttributeError):
        abi._load_lib()
    monkeypatch.setattr(abi, "_lib", None)
