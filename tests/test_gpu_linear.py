"""GPU parity of the HIP quantized linears against the golden vectors and the oracle.

Every comparison is bit-exact: the HIP kernels follow the reference's
summation order, so int8/int4 results must match the reference CPU kernels
byte for byte (fp32 outputs and bf16 outputs alike).  Calls go through the
C ABI (pilm_amd.ckernel -> ctypes -> libecpu.so), as piLM's Python does.
"""
from __future__ import annotations

import ctypes
import os
import sys

import numpy as np
import pytest

from pilm_amd import bindings as abi
from pilm_amd import synth as S
from tests import _golden as GV

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from pilm_amd import ckernel as ck  # noqa: E402


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def to_dev(a: np.ndarray, dev, bf16: bool = False):
    if bf16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def from_dev(t) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def run_gpu(fmt: str, x, w, s, dev, in_features=None):
    if fmt == "w8a32":
        return from_dev(ck.linear_w8a32(to_dev(x, dev), to_dev(w, dev), to_dev(s, dev)))
    xb = to_dev(x, dev, bf16=True)
    if fmt == "w8a16":
        return from_dev(ck.linear_w8a16_bf16(xb, to_dev(w, dev), to_dev(s, dev)))
    if fmt == "w4":
        return from_dev(ck.linear_w4a16_bf16(xb, to_dev(w, dev), to_dev(s, dev), in_features))
    fn = ck.linear_w4a16g32_bf16 if fmt == "w4g32" else ck.linear_w4a16g128_bf16
    return from_dev(fn(xb, to_dev(w, dev), to_dev(s, dev), in_features))


@pytest.mark.parametrize("case", GV.linear_cases(), ids=lambda c: c["name"])
def test_golden(case, dev):
    _say(f"[gpu] golden {case['name']}")
    y = run_gpu(case["fmt"], *GV.inputs(case), dev)
    GV.check_output(case, y)


SPLITS = [{"PILM_HIP_GQ": "0", "PILM_HIP_NSPLIT": "1"}, {"PILM_HIP_GQ": "0", "PILM_HIP_NSPLIT": "2"},
          {"PILM_HIP_GQ": "0", "PILM_HIP_NSPLIT": "3"}, {"PILM_HIP_GQ": "0", "PILM_HIP_NSPLIT": "16"},
          {"PILM_HIP_GQ": "0", "PILM_HIP_PL": "2"}, {"PILM_HIP_GQ": "0", "PILM_HIP_PL": "3"},
          {"PILM_HIP_GQ": "0", "PILM_HIP_PL": "8"}, {"PILM_HIP_GQ": "0", "PILM_HIP_PL": "2", "PILM_HIP_PG": "3"},
          {"PILM_HIP_GQ": "0", "PILM_HIP_PL": "8", "PILM_HIP_PG": "2"},
          {"PILM_HIP_GQ_P": "1"}, {"PILM_HIP_GQ_P": "2"}, {"PILM_HIP_GQ_P": "4"},
          {"PILM_HIP_GQ_P": "4", "PILM_HIP_GQ_D": "16"}, {"PILM_HIP_GQ_P": "8"},
          {"PILM_HIP_GQ_P": "8", "PILM_HIP_GQ_D": "8"}, {"PILM_HIP_GQ8": "0"}, {"PILM_HIP_GQ8": "1"},
          {"PILM_HIP_GQ8": "1", "PILM_HIP_GQ8_D": "4"}, {"PILM_HIP_GQ8": "1", "PILM_HIP_GQ8_D": "5"},
          {"PILM_HIP_GQ8": "1", "PILM_HIP_GQ8_D": "8"},
          {"PILM_HIP_BCAST_PL": "1"}, {"PILM_HIP_BCAST_PL": "3"}, {"PILM_HIP_BCAST_MT": "8"},
          {"PILM_HIP_BCAST_MT": "8", "PILM_HIP_BCAST_PL": "2"}, {"PILM_HIP_BCAST": "0"},
          {"PILM_HIP_BCAST": "0", "PILM_HIP_GQ": "0"}, {"PILM_HIP_BCAST_WIN": "1", "PILM_HIP_BCAST_MT": "4"},
          {"PILM_HIP_BCAST_WIN": "1", "PILM_HIP_BCAST_MT": "8"}, {"PILM_HIP_BCAST_WIN": "0"}]


@pytest.mark.parametrize("env", SPLITS, ids=lambda e: "_".join(f"{k[9:]}{v}" for k, v in e.items()))
def test_group_split_variants_identical(env, dev, monkeypatch):
    """Splitting K across waves (in LDS or in global memory; 64-row tiles,
    the 16- or 8-row group-quad tiles, or the small-M broadcast kernel) must
    not change a single bit."""
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    for prefix in ("config2_w4g128_M1", "config2_w4g128_M4", "w4g32_cancel", "w4g128_cancel"):
        for case in GV.linear_cases(prefix=prefix):
            if case["N"] > 20000:
                continue
            _say(f"[gpu] split {env} {case['name']}")
            GV.check_output(case, run_gpu(case["fmt"], *GV.inputs(case), dev))


ROW_PATHS = [{"PILM_HIP_CS": "0", "PILM_HIP_QUAD": "0", "PILM_HIP_ROWTILE": "64", "PILM_HIP_RING": "4"},
             {"PILM_HIP_CS": "0", "PILM_HIP_QUAD": "0", "PILM_HIP_ROWTILE": "64", "PILM_HIP_RING": "8"},
             {"PILM_HIP_CS": "0", "PILM_HIP_QUAD": "0", "PILM_HIP_ROWTILE": "64", "PILM_HIP_RING": "16"},
             {"PILM_HIP_CS": "0", "PILM_HIP_QUAD": "0", "PILM_HIP_ROWTILE": "32"},
             {"PILM_HIP_CS": "0", "PILM_HIP_QUAD": "0", "PILM_HIP_ROWTILE": "16"},
             {"PILM_HIP_CS": "0", "PILM_HIP_QUAD": "1", "PILM_HIP_RING": "4"},
             {"PILM_HIP_CS": "0", "PILM_HIP_QUAD": "1", "PILM_HIP_RING": "16"},
             {"PILM_HIP_CS": "2"}, {"PILM_HIP_CS": "4"},
             {"PILM_HIP_ROWS": "0"}, {"PILM_HIP_RBC": "0"}, {"PILM_HIP_RBC_MT": "4"}, {"PILM_HIP_RBC_MT": "5"},
             {"PILM_HIP_RBC_MT": "8"},
             {"PILM_HIP_W8B": "1", "PILM_HIP_W8B_ROWS": "16"}, {"PILM_HIP_W8B": "1", "PILM_HIP_W8B_ROWS": "32"},
             {"PILM_HIP_W8B": "1", "PILM_HIP_W8B_ROWS": "8"},
             {"PILM_HIP_W8B": "0"}, {"PILM_HIP_W4C8": "1"}, {"PILM_HIP_W4C8": "0"}]


@pytest.mark.parametrize("env", ROW_PATHS, ids=lambda e: "_".join(f"{k[9:]}{v}" for k, v in e.items()))
def test_row_format_paths_identical(env, dev, monkeypatch):
    """Per-row formats: every tile height and ring depth of the chain-split
    kernels (four waves per 64-row tile, four lanes per row, or two / four
    waves per 16-row tile), the one-wave-per-tile kernel, the byte-wave W8
    kernel (8-, 16- or 32-row tiles, or off) and the small-M row-broadcast
    kernel (4, 5 or 8 rows per wave, or off) give the same bits."""
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    for case in GV.linear_cases(max_elems=1 << 24):
        if case["fmt"] not in ("w8a32", "w8a16", "w4") or case["K"] % 256:
            continue
        _say(f"[gpu] rows {env} {case['name']}")
        GV.check_output(case, run_gpu(case["fmt"], *GV.inputs(case), dev))


def test_literal_path_identical(dev, monkeypatch):
    """The one-thread-per-output kernel gives the same bits on stripe-aligned shapes."""
    monkeypatch.setenv("PILM_HIP_LITERAL", "1")
    for case in GV.linear_cases(max_elems=1 << 22):
        if case["K"] % 128:
            continue
        _say(f"[gpu] literal {case['name']}")
        GV.check_output(case, run_gpu(case["fmt"], *GV.inputs(case), dev))


@pytest.mark.parametrize("fmt", ["w8a32", "w8a16", "w4", "w4g32", "w4g128"])
def test_fresh_shapes_against_oracle(fmt, dev):
    from oracle import oracle as O
    gen = GV._gen()
    rng = np.random.default_rng(2024)
    for trial in range(12):
        m = int(rng.choice([1, 2, 4, 5, 7, 16, 33]))
        n = int(rng.integers(1, 700))
        k = int(rng.choice([128, 256, 640, 1024, 2048, 4096, 96, 130, 1001]))
        _say(f"[gpu] oracle {fmt} M={m} N={n} K={k}")
        x, w, s = gen.make_inputs(fmt, m, n, k, 777 + trial)
        y = run_gpu(fmt, x, w, s, dev)
        ref = gen.run(fmt, x, w, s, "oracle")
        assert np.array_equal(y.view(np.uint8), ref.view(np.uint8)), (fmt, m, n, k)


@pytest.mark.parametrize("fmt", ["w4g32", "w4g128"])
def test_long_rows_group_quad(fmt, dev):
    """K = 12288 (Qwen3-8B down_proj): 24 KB of activations per tile beside
    the rings (group 32: 48 KB of scales and block sums as well, so fewer
    waves per tile, and launches of fewer activation rows); the small-M
    kernel's windowed fold where its parked block sums would not fit (group
    32, K = 4096 and 12288); the bits stay the oracle's."""
    gen = GV._gen()
    for m, n, k in ((1, 200, 12288), (2, 37, 12288), (4, 64, 12288), (5, 300, 12288), (8, 24, 12288),
                    (5, 1024, 4096), (7, 90, 4096), (16, 100, 12288), (24, 70, 12288), (13, 500, 4096)):
        _say(f"[gpu] long rows {fmt} M={m} N={n} K={k}")
        x, w, s = gen.make_inputs(fmt, m, n, k, 4242 + m)
        y = run_gpu(fmt, x, w, s, dev)
        ref = gen.run(fmt, x, w, s, "oracle")
        assert np.array_equal(y.view(np.uint8), ref.view(np.uint8)), (fmt, m, n, k)


@pytest.mark.parametrize("fmt", ["w8a32", "w8a16", "w4"])
def test_small_m_row_formats(fmt, dev):
    """Per-row formats at 3 <= M < 64 (MTP verify, short prefill), and M = 2
    beyond 8192 rows: the row-broadcast kernel against the oracle, ragged N
    and partial m-groups."""
    gen = GV._gen()
    for m, n, k in ((3, 50, 1024), (5, 300, 2048), (8, 17, 256), (9, 64, 4096), (16, 130, 512), (33, 40, 768),
                    (2, 8200, 256)):
        _say(f"[gpu] small-M {fmt} M={m} N={n} K={k}")
        x, w, s = gen.make_inputs(fmt, m, n, k, 9100 + m)
        y = run_gpu(fmt, x, w, s, dev)
        ref = gen.run(fmt, x, w, s, "oracle")
        assert np.array_equal(y.view(np.uint8), ref.view(np.uint8)), (fmt, m, n, k)


@pytest.mark.parametrize("fmt", ["w8a32", "w8a16", "w4", "w4g32", "w4g128"])
def test_m_boundaries(fmt, dev):
    """M around the kernel switches: 2 / 3 (group-quad or quad -> small-M
    kernels), 4 / 5 and 8 / 9 (m-groups of 4 and 8), 63 (the last exact M
    below the matrix cores); bit-exact against the oracle."""
    gen = GV._gen()
    for m in (2, 3, 4, 5, 8, 9, 63):
        n, k = 70, 512
        _say(f"[gpu] M boundary {fmt} M={m} N={n} K={k}")
        x, w, s = gen.make_inputs(fmt, m, n, k, 7300 + m)
        y = run_gpu(fmt, x, w, s, dev)
        ref = gen.run(fmt, x, w, s, "oracle")
        assert np.array_equal(y.view(np.uint8), ref.view(np.uint8)), (fmt, m, n, k)


def test_power_of_two_scale_full_size(dev):
    """Size-independent property at the lm_head shape: doubling the scales doubles every output."""
    n, k = 151936, 2048
    _say("[gpu] lm_head scale-doubling")
    x = to_dev(S.activations_bf16(11, 1, k), dev, bf16=True)
    w = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=dev)
    s = torch.rand((n, k // 128), device=dev) * 0.019 + 0.001
    y1 = ck.linear_w4a16g128_bf16(x, w, s).float()
    y2 = ck.linear_w4a16g128_bf16(x, w, s * 2).float()
    assert torch.equal(y2, y1 * 2)


def test_side_stream(dev):
    case = GV.linear_cases(prefix="config2_w4g128_M4_N4096")[0]
    x, w, s = GV.inputs(case)
    st = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(st):
        xd, wd, sd = to_dev(x, dev, bf16=True), to_dev(w, dev), to_dev(s, dev)
        y = ck.linear_w4a16g128_bf16(xd, wd, sd)
        out = from_dev(y)
    GV.check_output(case, out)


# ------------------------------------------------------------------ errors

def test_host_pointer_rejected(dev):
    x = np.zeros((1, 256), np.float32)
    w = np.zeros((8, 256), np.int8)
    s = np.ones(8, np.float32)
    c = np.zeros((1, 8), np.float32)
    rc = abi.linear_w8a32_ptr(x.ctypes.data, w.ctypes.data, s.ctypes.data, c.ctypes.data, 1, 8, 256)
    assert rc == abi.ECPU_ERR_PARAM
    assert "not device memory" in abi.last_error()


def test_null_rejected(dev):
    w = torch.zeros((8, 256), dtype=torch.int8, device=dev)
    rc = abi.linear_w8a32_ptr(0, w.data_ptr(), w.data_ptr(), w.data_ptr(), 1, 8, 256)
    assert rc == abi.ECPU_ERR_PARAM


def test_undersized_buffer_rejected(dev):
    lib = abi._load_lib()
    vt = lib.edevice_active()
    assert vt.contents.id == abi.EDEV_HIP
    alloc = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t)(vt.contents.alloc)
    free = ctypes.CFUNCTYPE(None, ctypes.c_void_p)(vt.contents.free)
    small = alloc(1 << 20, 256)
    big = alloc(64 << 20, 256)
    try:
        # W needs N*K = 2048*1024 bytes but only 1 MiB is allocated
        rc = abi.linear_w8a16_bf16_ptr(big, small, big, big, 1, 2048, 1024)
        assert rc == abi.ECPU_ERR_PARAM
        assert "allocation ends" in abi.last_error()
        rc = abi.linear_w8a16_bf16_ptr(big, big + (1 << 20), big + (4 << 20), big + (8 << 20), 1, 2048, 1024)
        assert rc == abi.ECPU_OK
        torch.cuda.synchronize()
    finally:
        free(small)
        free(big)


def test_wrapper_rejects_cpu_tensors(dev):
    x = torch.zeros((1, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        ck.linear_w4a16g128_bf16(x, torch.zeros((4, 64), dtype=torch.uint8, device=dev),
                                 torch.ones((4, 1), device=dev))


def test_gemm_and_swiglu(dev):
    rng = np.random.default_rng(5)
    a = rng.integers(-4, 5, size=(7, 33)).astype(np.float32)
    b = rng.integers(-4, 5, size=(9, 33)).astype(np.float32)
    out = ck.gemm_f32(to_dev(a, dev), to_dev(b, dev), transpose_b=True).cpu().numpy()
    assert np.array_equal(out, a @ b.T)
    out2 = ck.gemm_f32(to_dev(a, dev), to_dev(b.T.copy(), dev)).cpu().numpy()
    assert np.array_equal(out2, a @ b.T)
    g = rng.standard_normal(4096).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    gb, ub = S.f32_to_bf16_bits(g), S.f32_to_bf16_bits(u)
    y = S.bf16_bits_to_f32(from_dev(ck.swiglu_bf16(to_dev(gb, dev, True), to_dev(ub, dev, True))))
    gf, uf = S.bf16_bits_to_f32(gb).astype(np.float64), S.bf16_bits_to_f32(ub).astype(np.float64)
    ref = gf / (1 + np.exp(-gf)) * uf
    assert np.all(np.abs(y - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-30)
