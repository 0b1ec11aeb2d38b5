"""GPU: the argmax entry point that allocates nothing.

ekernel_linear_w8a16_bf16_argmax_noalloc keeps its intermediates in a
file-scope device array instead of allocated scratch.  Through the C ABI it
must give exactly what ekernel_linear_w8a16_bf16_argmax gives (index and the
bf16 value, bit for bit), on two calls in a row -- the second with fewer
rows, so the array still holds the first call's logits and partials -- with
host and with device outputs, and it must refuse N beyond its array.
"""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest

from pilm_amd import synth as S

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _inputs(dev, seed, n, k, ties=False):
    x = S.activations_bf16(seed, 1, k)
    w = S.weights_i8(seed + 1, n, k)
    s = S.scales_uniform(seed + 2, (n,), fp16_round=False)
    if ties:
        w[n // 2] = w[n // 5]
        s[n // 2] = s[n // 5]
    xd = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(dev)
    return xd, torch.from_numpy(w).to(dev), torch.from_numpy(s).to(dev)


def _call(lib, name, x, w, s, n, k, device_out):
    from pilm_amd import bindings as abi
    abi.set_stream(torch.cuda.current_stream().cuda_stream)
    desc = abi.EkernelLinearW8A32Desc(1, n, k)
    fn = getattr(lib, name)
    if device_out:
        idx = torch.full((1,), -1, dtype=torch.int64, device=x.device)
        val = torch.full((1,), float("nan"), dtype=torch.float32, device=x.device)
        rc = fn(ctypes.byref(desc), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(w.data_ptr()),
                ctypes.c_void_p(s.data_ptr()), ctypes.c_void_p(idx.data_ptr()), ctypes.c_void_p(val.data_ptr()), 6)
        assert rc == 0, abi.last_error()
        torch.cuda.synchronize()
        return int(idx.item()), np.float32(val.item()).view(np.uint32)
    i, v = ctypes.c_size_t(0), ctypes.c_float(0.0)
    rc = fn(ctypes.byref(desc), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(w.data_ptr()),
            ctypes.c_void_p(s.data_ptr()), ctypes.addressof(i), ctypes.addressof(v), 6)
    assert rc == 0, abi.last_error()
    return int(i.value), np.float32(v.value).view(np.uint32)


@pytest.mark.parametrize("epilogue", ["0", "1"], ids=["separate_argmax", "epilogue"])
@pytest.mark.parametrize("device_out", [False, True])
def test_noalloc_argmax_matches_the_allocating_entry(dev, device_out, epilogue, monkeypatch):
    from pilm_amd import bindings as abi
    monkeypatch.setenv("PILM_HIP_ARGMAX_EPILOGUE", epilogue)
    lib = abi._load_lib()
    # the first call sizes the array's use with a vocabulary-sized row, the
    # second (fewer rows, ties) reuses whatever the first left in it
    for seed, n, k, ties in ((11, 151936, 2048, False), (12, 4099, 512, True), (13, 32000, 4096, False)):
        x, w, s = _inputs(dev, seed, n, k, ties)
        _say(f"[gpu] no-alloc argmax N={n} K={k} device_out={device_out}")
        want = _call(lib, "ekernel_linear_w8a16_bf16_argmax", x, w, s, n, k, device_out)
        got = _call(lib, "ekernel_linear_w8a16_bf16_argmax_noalloc", x, w, s, n, k, device_out)
        assert got == want, (n, got, want)


def test_noalloc_argmax_refuses_rows_beyond_its_array(dev):
    from pilm_amd import bindings as abi
    lib = abi._load_lib()
    n, k = 262145, 8
    x = torch.zeros((1, k), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((n, k), dtype=torch.int8, device=dev)
    s = torch.ones((n,), dtype=torch.float32, device=dev)
    i, v = ctypes.c_size_t(0), ctypes.c_float(0.0)
    desc = abi.EkernelLinearW8A32Desc(1, n, k)
    rc = lib.ekernel_linear_w8a16_bf16_argmax_noalloc(ctypes.byref(desc), ctypes.c_void_p(x.data_ptr()),
                                                      ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(s.data_ptr()),
                                                      ctypes.addressof(i), ctypes.addressof(v), 6)
    assert rc == abi.ECPU_ERR_UNSUPPORTED
    assert "262144" in (abi.last_error() or "")
