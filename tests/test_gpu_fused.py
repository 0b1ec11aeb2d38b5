"""GPU parity of the fused epilogues against the golden vectors and the oracle.

  * ekernel_swiglu_bf16 on every bf16 gate value (the whole input domain of
    its expf), bit-exact;
  * ekernel_swiglu_w4a16_bf16 (the W4 SwiGLU MLP of one token), bit-exact,
    through the one-launch gate/up kernel and through the unfused fallback;
  * ekernel_linear_w8a16_bf16_argmax with host outputs (the reference
    binding's ctypes byref) and with device outputs, on golden cases, on
    logits holding NaN / +-inf / +-0 / ties, and on the Qwen3 lm_head shape.
Calls go through the C ABI (pilm_amd.ckernel / pilm_amd.bindings).
"""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest

from oracle import oracle as O
from pilm_amd import bindings as abi
from pilm_amd import synth as S
from tests import _golden as GV
from tests.test_oracle_fused import ARGMAX_KINDS, argmax_special_inputs

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from pilm_amd import ckernel as ck  # noqa: E402
from tests.test_gpu_linear import from_dev, to_dev  # noqa: E402


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _bits_equal(a, b) -> bool:
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


# ------------------------------------------------------------ SwiGLU

@pytest.mark.parametrize("case", GV.swiglu_bf16_cases(), ids=lambda c: c["name"])
def test_swiglu_bf16_every_gate(case, dev):
    g, u = GV.swiglu_bf16_inputs(case)
    _say(f"[gpu] swiglu_bf16 {case['name']}")
    y = from_dev(ck.swiglu_bf16(to_dev(g, dev, True), to_dev(u, dev, True)))
    GV.check_output(case, y)


def run_fused(ins, i_sz, dev, offset_x: bool = False):
    x, gu, gs, dw, ds = ins
    if offset_x:
        # A 2-byte offset leaves x unaligned for the stripe kernel: the
        # entry point must take its unfused path and give the same bits.
        buf = torch.empty((1, x.shape[1] + 1), dtype=torch.bfloat16, device=dev)
        buf[:, 1:].copy_(to_dev(x, dev, True))
        xd = buf[:, 1:]
        assert xd.data_ptr() % 16 != 0
        out = torch.empty((1, dw.shape[0]), dtype=torch.bfloat16, device=dev)
        held = [to_dev(a, dev) for a in (gu, gs, dw, ds)]
        ck._bind_stream(xd)
        rc = abi.swiglu_w4a16_bf16_ptr(xd.data_ptr(), *(t.data_ptr() for t in held),
                                       out.data_ptr(), 1, dw.shape[0], i_sz, x.shape[1], i_sz)
        torch.cuda.synchronize()
        assert rc == 0, abi.last_error()
        return from_dev(out)
    return from_dev(ck.swiglu_w4a16_bf16(to_dev(x, dev, True), to_dev(gu, dev), to_dev(gs, dev), to_dev(dw, dev),
                                         to_dev(ds, dev), i_sz))


@pytest.mark.parametrize("case", GV.swiglu_cases(), ids=lambda c: c["name"])
def test_fused_swiglu_golden(case, dev):
    _say(f"[gpu] swiglu_w4a16 {case['name']}")
    GV.check_output(case, run_fused(GV.swiglu_inputs(case), case["I"], dev))


@pytest.mark.parametrize("case", GV.swiglu_cases(max_weights=1 << 22), ids=lambda c: c["name"])
def test_fused_swiglu_unfused_path(case, dev):
    _say(f"[gpu] swiglu_w4a16 unaligned x {case['name']}")
    GV.check_output(case, run_fused(GV.swiglu_inputs(case), case["I"], dev, offset_x=True))


@pytest.mark.parametrize("ring", ["8", "16"])
def test_fused_swiglu_ring_depths(ring, dev, monkeypatch):
    monkeypatch.setenv("PILM_HIP_RING", ring)
    gen = GV._gen()
    for t, (h, i, k) in enumerate(((96, 256, 512), (64, 264, 256), (300, 2056, 1024), (128, 8200, 2048))):
        ins = gen.make_swiglu_inputs(h, i, k, 33000 + t)
        _say(f"[gpu] swiglu_w4a16 ring={ring} H={h} I={i} K={k}")
        assert _bits_equal(run_fused(ins, i, dev), O.swiglu_w4a16_bf16(*ins, i)), (h, i, k)


def test_fused_swiglu_rejects_like_reference(dev):
    gen = GV._gen()
    x, gu, gs, dw, ds = (to_dev(a, dev, j == 0) for j, a in enumerate(gen.make_swiglu_inputs(8, 16, 32, 1)))
    args = [x.data_ptr(), gu.data_ptr(), gs.data_ptr(), dw.data_ptr(), ds.data_ptr()]
    out = torch.empty((1, 8), dtype=torch.bfloat16, device=dev)
    ok = abi.swiglu_w4a16_bf16_ptr(*args, out.data_ptr(), 1, 8, 16, 32, 16)
    assert ok == 0
    assert abi.swiglu_w4a16_bf16_ptr(*args, out.data_ptr(), 2, 8, 16, 32, 16) == abi.ECPU_ERR_UNSUPPORTED
    assert abi.swiglu_w4a16_bf16_ptr(*args, out.data_ptr(), 1, 8, 16, 32, 15) == abi.ECPU_ERR_UNSUPPORTED
    assert abi.swiglu_w4a16_bf16_ptr(*args, 0, 1, 8, 16, 32, 16) == abi.ECPU_ERR_PARAM
    with pytest.raises(ValueError):
        ck.swiglu_w4a16_bf16(x.repeat(2, 1), gu, gs, dw, ds, 16)
    # a gate/up allocation too small for the descriptor is refused before launch
    with device_allocations(1 << 20, 64 << 20) as (small, big):
        # H=64, I=1024, K=2048: gate_up needs 2048 x 1024 bytes, 1 MiB is allocated
        rc = abi.swiglu_w4a16_bf16_ptr(big, small, big + (1 << 20), big + (2 << 20), big + (4 << 20),
                                       big + (5 << 20), 1, 64, 1024, 2048, 1024)
        assert rc == abi.ECPU_ERR_PARAM and "allocation ends" in abi.last_error()


class device_allocations:
    """hipMalloc'd buffers of the given sizes through the library's device
    vtable (each its own allocation, unlike the caching allocator's blocks)."""

    def __init__(self, *sizes):
        lib = abi._load_lib()
        vt = lib.edevice_active()
        assert vt.contents.id == abi.EDEV_HIP
        self._alloc = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t)(vt.contents.alloc)
        self._free = ctypes.CFUNCTYPE(None, ctypes.c_void_p)(vt.contents.free)
        self.sizes = sizes
        self.ptrs = []

    def __enter__(self):
        self.ptrs = [self._alloc(n, 256) for n in self.sizes]
        assert all(self.ptrs)
        return self.ptrs

    def __exit__(self, *exc):
        torch.cuda.synchronize()
        for p in self.ptrs:
            self._free(p)
        return False


# ------------------------------------------------------------ argmax

def argmax_gpu(x, w, s, dev, device_out: bool = False):
    xd, wd, sd = to_dev(x, dev, True), to_dev(w, dev), to_dev(s, dev)
    if device_out:
        idx, val = ck.linear_w8a16_bf16_argmax_device(xd, wd, sd)
        return int(idx.item()), float(val.item())
    xd2 = xd.reshape(1, -1)
    ck._bind_stream(xd2)
    rc, idx, val = abi.linear_w8a16_bf16_argmax_ptr(xd2.data_ptr(), wd.data_ptr(), sd.data_ptr(), 1, w.shape[0],
                                                    w.shape[1])
    assert rc == 0, abi.last_error()
    assert ck.linear_w8a16_bf16_argmax(xd, wd, sd) == idx
    return idx, val


def _same(a: tuple, b: tuple) -> bool:
    return a[0] == b[0] and np.float32(a[1]).tobytes() == np.float32(b[1]).tobytes()


@pytest.mark.parametrize("device_out", [False, True], ids=["host_out", "device_out"])
@pytest.mark.parametrize("case", GV.argmax_cases(), ids=lambda c: c["name"])
def test_argmax_golden(case, device_out, dev):
    _say(f"[gpu] argmax {case['name']} device_out={device_out}")
    got = argmax_gpu(*GV.argmax_inputs(case), dev, device_out)
    assert _same(got, (case["index"], case["value"])), (got, case["index"], case["value"])


@pytest.mark.parametrize("device_out", [False, True], ids=["host_out", "device_out"])
@pytest.mark.parametrize("kind", ARGMAX_KINDS)
@pytest.mark.parametrize("epilogue", ["0", "1"], ids=["separate_argmax", "epilogue"])
def test_argmax_special_logits(kind, device_out, epilogue, dev, monkeypatch):
    """The GEMV + argmax kernel pair (default), and the GEMV with the argmax
    epilogue (K = 128: whole 128-byte stripes)."""
    monkeypatch.setenv("PILM_HIP_ARGMAX_EPILOGUE", epilogue)
    x, w, s = argmax_special_inputs(kind, 4100 + ARGMAX_KINDS.index(kind), k=128)
    _say(f"[gpu] argmax special {kind} epilogue={epilogue} device_out={device_out}")
    assert _same(argmax_gpu(x, w, s, dev, device_out), O.linear_w8a16_bf16_argmax(x, w, s))


@pytest.mark.parametrize("epilogue", ["0", "1"], ids=["separate_argmax", "epilogue"])
def test_argmax_many_workgroups_and_ties(epilogue, dev, monkeypatch):
    """Sizes that spread the logits over 1..2374 workgroups, with the maximum
    placed in the last, the first and a middle workgroup and repeated."""
    monkeypatch.setenv("PILM_HIP_ARGMAX_EPILOGUE", epilogue)
    k = 128
    rng = np.random.default_rng(9)
    for n in (1, 7, 2048, 2049, 4097, 65536 + 3, 151936):
        x = S.activations_bf16(int(n) + 11, 1, k)
        w = S.weights_i8(int(n) + 12, n, k)
        s = S.scales_uniform(int(n) + 13, (n,), fp16_round=False)
        xf = S.bf16_bits_to_f32(x[0])
        top = (np.sign(xf) * 127).astype(np.int8)
        for where in sorted({n - 1, 0, n // 2, int(rng.integers(0, n))}):
            w2, s2 = w.copy(), s.copy()
            w2[where], s2[where] = top, np.float32(2.0)
            if where + 3 < n:
                w2[where + 3], s2[where + 3] = top, np.float32(2.0)   # a tie after it
            _say(f"[gpu] argmax N={n} max at {where}")
            exp = O.linear_w8a16_bf16_argmax(x, w2, s2)
            assert exp[0] == where
            assert _same(argmax_gpu(x, w2, s2, dev), exp)
            assert _same(argmax_gpu(x, w2, s2, dev, True), exp)


@pytest.mark.parametrize("epilogue", ["0", "1"], ids=["separate_argmax", "epilogue"])
@pytest.mark.parametrize("k", [2048, 4096], ids=["qwen3_1p7b", "qwen3_8b"])
def test_argmax_lm_head_shape(k, epilogue, dev, monkeypatch):
    """The Qwen3 lm_head (151936 rows) of the two decode configurations, with
    the argmax as the GEMV's epilogue and as a kernel of its own."""
    monkeypatch.setenv("PILM_HIP_ARGMAX_EPILOGUE", epilogue)
    n = 151936
    x = S.activations_bf16(8100 + k, 1, k)
    w = S.weights_i8(8101 + k, n, k)
    s = S.scales_uniform(8102 + k, (n,), fp16_round=False)
    _say(f"[gpu] argmax lm_head N={n} K={k}")
    exp = O.linear_w8a16_bf16_argmax(x, w, s)
    assert _same(argmax_gpu(x, w, s, dev), exp)
    assert _same(argmax_gpu(x, w, s, dev, True), exp)


def test_argmax_rejects_like_reference(dev):
    x = torch.zeros((2, 64), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((8, 64), dtype=torch.int8, device=dev)
    s = torch.ones((8,), dtype=torch.float32, device=dev)
    rc, _, _ = abi.linear_w8a16_bf16_argmax_ptr(x.data_ptr(), w.data_ptr(), s.data_ptr(), 2, 8, 64)
    assert rc == abi.ECPU_ERR_UNSUPPORTED
    rc, _, _ = abi.linear_w8a16_bf16_argmax_ptr(x.data_ptr(), w.data_ptr(), s.data_ptr(), 1, 0, 64)
    assert rc == abi.ECPU_ERR_UNSUPPORTED
    with pytest.raises(ValueError):
        ck.linear_w8a16_bf16_argmax(x, w, s)
    with device_allocations(1 << 20, 8 << 20) as (small, big):
        # W needs 4096 x 512 bytes, 1 MiB is allocated
        rc, _, _ = abi.linear_w8a16_bf16_argmax_ptr(big, small, big + (1 << 20), 1, 4096, 512)
        assert rc == abi.ECPU_ERR_PARAM and "allocation ends" in abi.last_error()
