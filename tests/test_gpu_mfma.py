"""GPU: the matrix-core dequant-GEMM taken by M >= 64 activation rows.

This path is not bit-identical to the reference (fp16 operands, fp32 sums in
another order); the tolerance for it is a 1e-2 maximum relative error,
measured per output row against that row's largest magnitude:

    max_n |y[m,n] - ref[m,n]|  <=  1e-2 * max_n |ref[m,n]|      for every m

where ref is the oracle (bit-identical to the reference CPU kernels).  The
typical error is far smaller, so the tests also bound the RMS error at 3e-3 of
the RMS output -- a misplaced nibble, scale or row would break both bounds.
Calls go through the C ABI like piLM's own (pilm_amd.ckernel).
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

from pilm_amd import synth as S
from tests import _golden as GV

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from tests.test_gpu_linear import run_gpu  # noqa: E402

TOL_MAX_REL = 1e-2     # the MFMA path tolerance, per output row
TOL_RMS_REL = 3e-3

FMTS = ["w8a32", "w8a16", "w4", "w4g32", "w4g128"]


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def as_f32(fmt: str, y: np.ndarray) -> np.ndarray:
    return y.astype(np.float64) if fmt == "w8a32" else S.bf16_bits_to_f32(y).astype(np.float64)


def check_close(fmt, y, ref, what):
    yf, rf = as_f32(fmt, y), as_f32(fmt, ref)
    assert np.all(np.isfinite(yf)), what
    err = np.abs(yf - rf)
    rowmax = np.abs(rf).max(axis=1)
    bad = err.max(axis=1) > TOL_MAX_REL * rowmax
    assert not bad.any(), f"{what}: rows {np.nonzero(bad)[0][:8]} exceed {TOL_MAX_REL} (max rel {(err.max(axis=1) / np.maximum(rowmax, 1e-30)).max():.3g})"
    rms = np.sqrt((err ** 2).mean()) / max(np.sqrt((rf ** 2).mean()), 1e-30)
    assert rms <= TOL_RMS_REL, f"{what}: rms relative error {rms:.3g}"
    return float((err.max(axis=1) / np.maximum(rowmax, 1e-30)).max())


SHAPES = [(64, 32, 64), (64, 100, 192), (80, 200, 512), (128, 128, 1024), (200, 513, 320), (256, 1000, 2048),
          (129, 64, 4096)]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_mfma_against_oracle(fmt, shape, dev):
    m, n, k = shape
    gen = GV._gen()
    x, w, s = gen.make_inputs(fmt, m, n, k, 4242 + m + n + k)
    _say(f"[gpu] mfma {fmt} M={m} N={n} K={k}")
    y = run_gpu(fmt, x, w, s, dev)
    ref = gen.run(fmt, x, w, s, "oracle")
    check_close(fmt, y, ref, f"{fmt} {shape}")


@pytest.mark.parametrize("fmt", FMTS)
def test_mfma_config3_shape(fmt, dev):
    """One prefill shape of the 8B model (gate/up rows, K = hidden) at M=256."""
    m, n, k = 256, 2048, 4096
    gen = GV._gen()
    x, w, s = gen.make_inputs(fmt, m, n, k, 99)
    _say(f"[gpu] mfma config3 {fmt} M={m} N={n} K={k}")
    y = run_gpu(fmt, x, w, s, dev)
    ref = gen.run(fmt, x, w, s, "oracle")
    check_close(fmt, y, ref, f"{fmt} config3")


@pytest.mark.parametrize("shape", SHAPES + [(256, 2048, 4096)], ids=lambda s: "x".join(map(str, s)))
def test_mfma_w8a16_both_operand_types(shape, dev, monkeypatch):
    """W8A16 runs on bf16 MFMAs by default (the bf16 activations as they are,
    each int8 weight converted exactly) and on fp16 MFMAs after the
    activation pass with PILM_HIP_MFMA_BF16=0.  Either way every product is
    exact and only the fp32 order of the sums differs from the reference, so
    each output lies within one bf16 rounding step of the oracle's
    (2^-7 |ref| covers a step on either side) except where the row's sums
    cancel (1e-3 of the row's largest output)."""
    m, n, k = shape
    gen = GV._gen()
    x, w, s = gen.make_inputs("w8a16", m, n, k, 515 + m + n + k)
    ref = gen.run("w8a16", x, w, s, "oracle")
    rf = as_f32("w8a16", ref)
    for bf16 in ("1", "0"):
        monkeypatch.setenv("PILM_HIP_MFMA_BF16", bf16)
        _say(f"[gpu] mfma w8a16 bf16={bf16} M={m} N={n} K={k}")
        y = run_gpu("w8a16", x, w, s, dev)
        check_close("w8a16", y, ref, f"w8a16 bf16={bf16} {shape}")
        err = np.abs(as_f32("w8a16", y) - rf)
        bound = 2.0 ** -7 * np.abs(rf) + 1e-3 * np.abs(rf).max(axis=1, keepdims=True)
        assert (err <= bound).all(), f"bf16={bf16}: {(err > bound).sum()} outputs beyond one bf16 step"


@pytest.mark.parametrize("fmt", ["w8a16", "w4g128"])
def test_below_threshold_stays_exact(fmt, dev, monkeypatch):
    """M below the threshold, or the threshold disabled, keeps the exact kernels."""
    gen = GV._gen()
    x, w, s = gen.make_inputs(fmt, 63, 96, 512, 7)
    _say(f"[gpu] exact M=63 {fmt}")
    y = run_gpu(fmt, x, w, s, dev)
    assert np.array_equal(y.view(np.uint8), gen.run(fmt, x, w, s, "oracle").view(np.uint8))
    monkeypatch.setenv("PILM_HIP_MFMA_MIN_M", "0")
    x, w, s = gen.make_inputs(fmt, 128, 96, 512, 8)
    _say(f"[gpu] exact M=128 {fmt} (matrix cores off)")
    y = run_gpu(fmt, x, w, s, dev)
    assert np.array_equal(y.view(np.uint8), gen.run(fmt, x, w, s, "oracle").view(np.uint8))


def test_mfma_zero_and_sign_extremes(dev):
    """All-(-8) int4 weights, all-(-128) int8 weights and zero activations."""
    gen = GV._gen()
    for fmt in FMTS:
        x, w, s = gen.make_inputs(fmt, 96, 64, 256, 5, special="min_w")
        _say(f"[gpu] mfma min_w {fmt}")
        check_close(fmt, run_gpu(fmt, x, w, s, dev), gen.run(fmt, x, w, s, "oracle"), f"{fmt} min_w")
        x, w, s = gen.make_inputs(fmt, 96, 64, 256, 6, special="zero_x")
        y = as_f32(fmt, run_gpu(fmt, x, w, s, dev))
        assert np.all(y == 0.0), fmt


@pytest.mark.parametrize("splits", ["1", "3", "7"])
def test_mfma_split_k(splits, dev, monkeypatch):
    """Split K (fp32 partials summed in split order): same tolerance, and the
    same bits on every run."""
    monkeypatch.setenv("PILM_HIP_MFMA_SPLITS", splits)
    gen = GV._gen()
    for fmt in FMTS:
        x, w, s = gen.make_inputs(fmt, 96, 160, 1024, 31)
        _say(f"[gpu] mfma splits={splits} {fmt}")
        y = run_gpu(fmt, x, w, s, dev)
        check_close(fmt, y, gen.run(fmt, x, w, s, "oracle"), f"{fmt} splits={splits}")
        assert np.array_equal(y.view(np.uint8), run_gpu(fmt, x, w, s, dev).view(np.uint8)), "not deterministic"


@pytest.mark.parametrize("fmt", ["w8a16", "w4g128", "w4"])
@pytest.mark.parametrize("nseq", [12, 16])
def test_continuous_batching_verify(fmt, nseq, dev):
    """MTP verify under continuous batching (src/engine.py:416-545,
    scheduler.py:70-178): every sequence's 1 + 4 draft rows go into one call,
    M = 5 * nseq, compared with the oracle.  Below the matrix-core threshold
    (12 sequences, M = 60) the call is bit-identical to it; from the threshold
    on (16 sequences, M = 80) the matrix-core call is within its tolerance and
    the same call forced onto the exact kernels (threshold 0, what the batched
    decoder's verify step does) is bit-identical again."""
    from pilm_amd import bindings as abi
    gen = GV._gen()
    n, k = 1024, 4096          # Qwen3-8B k_proj
    x, w, s = gen.make_inputs(fmt, 5 * nseq, n, k, 9500 + nseq)
    _say(f"[gpu] batched verify {fmt} sequences={nseq} M={5 * nseq}")
    y = run_gpu(fmt, x, w, s, dev)
    ref = gen.run(fmt, x, w, s, "oracle")
    if 5 * nseq < 64:
        assert np.array_equal(y.view(np.uint8), ref.view(np.uint8)), fmt
        return
    check_close(fmt, y, ref, f"{fmt} batched M={5 * nseq}")
    prev = abi.matrix_core_min_rows()
    abi.set_matrix_core_min_rows(0)
    try:
        y0 = run_gpu(fmt, x, w, s, dev)
    finally:
        abi.set_matrix_core_min_rows(prev)
    assert np.array_equal(y0.view(np.uint8), ref.view(np.uint8)), f"{fmt} exact kernels at M={5 * nseq}"


@pytest.mark.parametrize("bm,wm", [("64", "1"), ("64", "2"), ("128", "1"), ("128", "2"), ("256", "2")])
@pytest.mark.parametrize("fmt", ["w8a32", "w4g128", "w4g32", "w4"])
def test_mfma_tile_heights(bm, wm, fmt, dev, monkeypatch):
    """Every output-tile height (64, 128, 256 rows of M) and wave layout
    (1 x 4 or 2 x 2) stays within the matrix-core tolerance, ragged M and N
    included."""
    monkeypatch.setenv("PILM_HIP_MFMA_BM", bm)
    monkeypatch.setenv("PILM_HIP_MFMA_WM", wm)
    gen = GV._gen()
    m, n, k = 300, 1000, 2048
    _say(f"[gpu] mfma tile {bm} waves {wm} {fmt} {m}x{n}x{k}")
    x, w, s = gen.make_inputs(fmt, m, n, k, 8800 + int(bm) + int(wm))
    y = run_gpu(fmt, x, w, s, dev)
    ref = gen.run(fmt, x, w, s, "oracle")
    check_close(fmt, y, ref, f"{fmt} BM={bm} WM={wm}")


# ----------------------------------------------------- range of the fp16 operands

RANGE_CASES = {
    # name: (activation factor, scale factor)
    "tiny_x": (1e-20, 1.0),          # below fp16's normal range
    "large_x": (1e30, 1.0),          # far beyond 65504
    "tiny_scales": (1.0, 1e-7),      # group scale x weight in the fp16 subnormals
    "large_scales": (1.0, 1e6),      # group scale x weight beyond 65504
    "mixed_rows": (None, 1.0),       # each activation row at its own magnitude, 1e-20 .. 1e20
}


def _scaled_inputs(fmt, case, m=96, n=160, k=1024, seed=77):
    gen = GV._gen()
    x, w, s = gen.make_inputs(fmt, m, n, k, seed)
    xs, ss = RANGE_CASES[case]
    xf = x.astype(np.float64) if fmt == "w8a32" else S.bf16_bits_to_f32(x).astype(np.float64)
    if xs is None:
        xf = xf * (10.0 ** np.linspace(-20, 20, m))[:, None]
    else:
        xf = xf * xs
    x = xf.astype(np.float32) if fmt == "w8a32" else S.f32_to_bf16_bits(xf.astype(np.float32))
    return x, w, (s.astype(np.float64) * ss).astype(np.float32)


@pytest.mark.parametrize("splits", ["auto", "3"])
@pytest.mark.parametrize("case", list(RANGE_CASES))
@pytest.mark.parametrize("fmt", FMTS)
def test_mfma_operand_range(fmt, case, splits, dev, monkeypatch):
    """Activations and scales far outside fp16's range keep the matrix-core
    tolerance: each activation row and each weight row is scaled by a power
    of two into range before the fp16 conversion and scaled back exactly."""
    if splits != "auto":
        monkeypatch.setenv("PILM_HIP_MFMA_SPLITS", splits)
    x, w, s = _scaled_inputs(fmt, case)
    gen = GV._gen()
    _say(f"[gpu] mfma range {fmt} {case} splits={splits}")
    y = run_gpu(fmt, x, w, s, dev)
    check_close(fmt, y, gen.run(fmt, x, w, s, "oracle"), f"{fmt} {case}")


@pytest.mark.parametrize("special", ["large_x", "denormal_x"])
@pytest.mark.parametrize("fmt", FMTS)
def test_mfma_golden_extremes_at_prefill_rows(fmt, special, dev):
    """The golden files' extreme activations (x 1e30, x 1e-39 subnormal),
    generated the same way at M = 96.  Subnormal outputs carry only a few bits
    in either order of summation, so the bound adds K subnormal steps."""
    gen = GV._gen()
    m, n, k = 96, 70, 256
    x, w, s = gen.make_inputs(fmt, m, n, k, 4711, special)
    _say(f"[gpu] mfma golden extreme {fmt} {special}")
    y = as_f32(fmt, run_gpu(fmt, x, w, s, dev))
    ref = as_f32(fmt, gen.run(fmt, x, w, s, "oracle"))
    assert np.all(np.isfinite(y))
    sub = k * 2.0 ** -149 + (0.0 if fmt == "w8a32" else 2.0 ** -133)
    tol = TOL_MAX_REL * np.abs(ref).max(axis=1, keepdims=True) + sub
    bad = np.abs(y - ref) > tol
    assert not bad.any(), f"{bad.sum()} outputs beyond tolerance"


@pytest.mark.parametrize("fmt", ["w8a16", "w4g128", "w4"])
def test_matrix_core_threshold_setter(fmt, dev):
    """ecpu_hip_set_matrix_core_min_rows: above M every row stays bit-exact;
    0 never takes the matrix cores; a negative value returns to the default."""
    from pilm_amd import bindings as abi
    gen = GV._gen()
    x, w, s = gen.make_inputs(fmt, 80, 256, 1024, 321)
    ref = gen.run(fmt, x, w, s, "oracle")
    try:
        for rows in (81, 0):
            abi.set_matrix_core_min_rows(rows)
            assert abi.matrix_core_min_rows() == rows
            _say(f"[gpu] threshold {rows} {fmt} M=80")
            assert np.array_equal(run_gpu(fmt, x, w, s, dev).view(np.uint8), ref.view(np.uint8))
    finally:
        abi.set_matrix_core_min_rows(-1)
    assert abi.matrix_core_min_rows() == 64
    check_close(fmt, run_gpu(fmt, x, w, s, dev), ref, f"{fmt} default threshold")


# ------------------------------------------------- configuration 3 at full size

CONFIG3_SHAPES = [(8192, 4096), (24576, 4096), (4096, 12288), (151936, 4096)]   # Qwen3-8B q / gate_up / down / lm_head
CONFIG3_M = [64, 256, 1024, 2048]
_C3_CACHE: dict = {}


def _c3_weights(fmt, n, k, dev):
    """Seeded device weights of the configuration's distributions (int8
    uniform in [-127, 127] or packed int4 bytes uniform; scales ~U(0.001,
    0.02), group scales rounded through fp16), kept across the M values."""
    key = (fmt, n, k)
    if key not in _C3_CACHE:
        _C3_CACHE.clear()
        torch.cuda.empty_cache()
        g = torch.Generator(device=dev)
        g.manual_seed(n * 7 + k)
        if fmt == "w8a32":
            w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev, generator=g)
            s = torch.rand((n,), device=dev, generator=g) * 0.019 + 0.001
        else:
            w = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=dev, generator=g)
            s = (torch.rand((n, k // 128), device=dev, generator=g) * 0.019 + 0.001).half().float()
        _C3_CACHE[key] = (w, s)
    return _C3_CACHE[key]


def _c3_run(fmt, x, w, s, k):
    from pilm_amd import ckernel as ck
    if fmt == "w8a32":
        return ck.linear_w8a32(x, w, s)
    return ck.linear_w4a16g128_bf16(x, w, s, k)


@pytest.mark.parametrize("m", CONFIG3_M)
@pytest.mark.parametrize("n,k", CONFIG3_SHAPES, ids=lambda v: str(v))
@pytest.mark.parametrize("fmt", ["w8a32", "w4g128"])
def test_config3_full_shapes(fmt, n, k, m, dev):
    """The prefill / verify GEMM at the Qwen3-8B shapes and M of the
    configuration: 128 sampled weight rows (every activation row) against the
    oracle on the sliced weights, within the matrix-core tolerance; over the
    whole output, doubling every scale doubles every output exactly (a power
    of two passes through the fp16 operands and the epilogue unchanged)."""
    w, s = _c3_weights(fmt, n, k, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(m)
    x = torch.randn((m, k), device=dev, generator=g)
    if fmt != "w8a32":
        x = x.to(torch.bfloat16)
    _say(f"[gpu] config3 {fmt} M={m} N={n} K={k}")
    y = _c3_run(fmt, x, w, s, k)
    rows = torch.randperm(n, generator=torch.Generator().manual_seed(n + m))[:128].sort().values
    xs = x.cpu().numpy() if fmt == "w8a32" else x.view(torch.int16).cpu().numpy().view(np.uint16)
    ws, ss = w[rows.to(dev)].cpu().numpy(), s[rows.to(dev)].cpu().numpy()
    gen = GV._gen()
    ref = gen.run(fmt, xs, ws, ss, "oracle")
    yr = y[:, rows.to(dev)]
    got = yr.cpu().numpy() if fmt == "w8a32" else yr.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    check_close(fmt, got, ref, f"{fmt} {m}x{n}x{k} sampled rows")
    y2 = _c3_run(fmt, x, w, s * 2, k)
    if fmt == "w8a32":
        assert torch.equal(y2, y * 2)
    else:
        assert torch.equal(y2.float(), y.float() * 2)
    del y, y2


@pytest.mark.parametrize("fmt", ["w8a32", "w4g128"])
def test_config3_zero_rows(fmt, dev):
    """Zero weight rows give exactly zero outputs in a full-size call."""
    n, k, m = 24576, 4096, 256
    w, s = _c3_weights(fmt, n, k, dev)
    w = w.clone()
    zero = torch.arange(0, n, 997, device=dev)
    w[zero] = 0 if fmt == "w8a32" else 0x00
    x = torch.randn((m, k), device=dev)
    if fmt != "w8a32":
        x = x.to(torch.bfloat16)
    _say(f"[gpu] config3 zero rows {fmt}")
    y = _c3_run(fmt, x, w, s, k).float()
    assert torch.all(y[:, zero] == 0)
    assert torch.count_nonzero(y) > 0.99 * (y.numel() - m * zero.numel())
