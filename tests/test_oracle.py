"""Pins the CPU oracle (oracle/oracle.c + oracle/oracle.py).

The oracle is what the HIP kernels are compared with, so it is checked first:
  * against the golden vectors written from the reference's own kernels.c;
  * against the reference library built from source, on fresh seeds, when
    oracle/_ref has been built (it needs the reference sources);
  * against mathematics that fixes the answer independently of any summation
    order (exact integer dot products, single-term sums, power-of-two scaling,
    an fp64 error bound);
  * and each plausible mistake, planted in a separate build of the oracle,
    must be rejected by the golden vectors.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from pilm_amd import synth as S
from tests import _golden as GV


def _run(fmt, x, w, s, impl="oracle"):
    if fmt == "w8a32":
        return O.linear_w8a32(x, w, s, impl=impl)
    if fmt == "w8a16":
        return O.linear_w8a16_bf16(x, w, s, impl=impl)
    if fmt == "w4":
        return O.linear_w4a16_bf16(x, w, s, impl=impl)
    return O.linear_w4a16g_bf16(x, w, s, 32 if fmt == "w4g32" else 128, impl=impl)


def test_golden_inputs_regenerate():
    """The seeded generator still produces the exact inputs the vectors were made from."""
    for c in GV.linear_cases(max_elems=1 << 22)[::7]:
        assert GV.sha(*GV.inputs(c)) == c["input_sha256"], c["name"]


@pytest.mark.parametrize("case", GV.linear_cases(max_elems=1 << 24), ids=lambda c: c["name"])
def test_oracle_matches_golden(case):
    y = _run(case["fmt"], *GV.inputs(case))
    GV.check_output(case, y)


def test_oracle_matches_golden_large():
    """Full-size configuration shapes (lm_head 151936 x 2048 etc.)."""
    for case in GV.linear_cases(prefix="config"):
        if case["M"] * case["N"] * case["K"] <= 1 << 24:
            continue
        if case["M"] > 4 and case["N"] > 100000:
            continue  # the M=16 lm_head case alone is ~5 G FMAs; covered on the GPU
        GV.check_output(case, _run(case["fmt"], *GV.inputs(case)))


@pytest.mark.parametrize("case", GV.argmax_cases(), ids=lambda c: c["name"])
def test_oracle_argmax_matches_golden(case):
    idx, val = O.linear_w8a16_bf16_argmax(*GV.argmax_inputs(case))
    assert idx == case["index"]
    assert val == case["value"]


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (reference sources absent)")
def test_oracle_matches_reference_build_fresh_seeds():
    rng = np.random.default_rng(12345)
    for trial in range(120):
        fmt = ("w8a32", "w8a16", "w4", "w4g32", "w4g128")[trial % 5]
        m = int(rng.integers(1, 6))
        n = int(rng.integers(1, 40))
        k = int(rng.integers(1, 700))
        x, w, s = GV._gen().make_inputs(fmt, m, n, k, 90000 + trial)
        a = _run(fmt, x, w, s)
        b = _run(fmt, x, w, s, impl="ref")
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), (fmt, m, n, k)


# ------------------------------------------------------------ planted mistakes

PLANTS = {
    1: "tails without FMA",
    2: "hsum in lane order",
    3: "group fold without FMA",
    4: "nibble order swapped",
    5: "zero-point decode",
    6: "bf16 truncation",
    7: "single int4 accumulator",
}


@pytest.mark.parametrize("variant", sorted(PLANTS), ids=lambda v: PLANTS[v])
def test_golden_vectors_reject_planted_mistake(variant):
    cases = sorted(GV.linear_cases(max_elems=1 << 24), key=lambda c: c["M"] * c["N"] * max(c["K"], 1))
    for case in cases:
        y = _run(case["fmt"], *GV.inputs(case), impl=variant)
        if GV.sha(y) != case["output_sha256"]:
            return
    pytest.fail(f"planted mistake {variant} ({PLANTS[variant]}) passed every golden vector")


# ------------------------------------------------------------ closed forms

def test_small_integer_inputs_are_exact():
    """Integer activations and unit scales: every partial sum is an exactly
    representable integer, so any summation order gives the integer dot."""
    rng = np.random.default_rng(7)
    for k in (8, 33, 256, 1000):
        n = 9
        xi = rng.integers(-8, 9, size=(2, k))
        w8 = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
        ones = np.ones(n, np.float32)
        y = O.linear_w8a32(xi.astype(np.float32), w8, ones)
        assert np.array_equal(y, (xi @ w8.astype(np.int64).T).astype(np.float32))
        yb = O.linear_w8a16_bf16(S.f32_to_bf16_bits(xi.astype(np.float32)), w8, ones)
        exp = S.f32_to_bf16_bits((xi @ w8.astype(np.int64).T).astype(np.float32))
        assert np.array_equal(yb, exp)
        w4 = S.weights_i4_packed(k, n, k)
        q = O.unpack_i4_rows_to_i8(w4, k).astype(np.int64)
        y4 = O.linear_w4a16_bf16(S.f32_to_bf16_bits(xi.astype(np.float32)), w4, ones)
        assert np.array_equal(y4, S.f32_to_bf16_bits((xi @ q.T).astype(np.float32)))
        g = np.ones((n, (k + 127) // 128), np.float32)
        y4g = O.linear_w4a16g_bf16(S.f32_to_bf16_bits(xi.astype(np.float32)), w4, g, 128)
        assert np.array_equal(y4g, S.f32_to_bf16_bits((xi @ q.T).astype(np.float32)))


def test_single_nonzero_term():
    """One nonzero activation: y[n] = a * w[n, k0] * scale[n], one rounding."""
    k, n = 300, 13
    for k0 in (0, 7, 8, 150, 299):
        x = np.zeros((1, k), np.float32)
        x[0, k0] = 1.375
        w = S.weights_i8(k0, n, k)
        s = S.scales_uniform(k0, (n,), fp16_round=False)
        y = O.linear_w8a32(x, w, s)
        exp = (np.float32(1.375) * w[:, k0].astype(np.float32)) * s
        assert np.array_equal(y[0], exp.astype(np.float32))


def test_power_of_two_scale_is_exact():
    """Doubling every scale doubles every output bit-exactly."""
    for fmt in ("w8a32", "w8a16", "w4", "w4g32", "w4g128"):
        x, w, s = GV._gen().make_inputs(fmt, 3, 37, 515, 31)
        y1 = _run(fmt, x, w, s).astype(np.float32) if fmt == "w8a32" else S.bf16_bits_to_f32(_run(fmt, x, w, s))
        y2 = _run(fmt, x, w, (s * 2).astype(np.float32))
        y2 = y2 if fmt == "w8a32" else S.bf16_bits_to_f32(y2)
        assert np.array_equal(y2, y1 * 2), fmt


def test_within_fp64_error_bound():
    """|y - y64| <= gamma_K * sum|a w| * scale (+ bf16 rounding), gamma_K = K u / (1 - K u)."""
    u = 2.0 ** -24
    for fmt in ("w8a32", "w4", "w4g128"):
        m, n, k = 2, 50, 1024
        x, w, s = GV._gen().make_inputs(fmt, m, n, k, 77)
        xf = x.astype(np.float64) if fmt == "w8a32" else S.bf16_bits_to_f32(x).astype(np.float64)
        if fmt == "w8a32":
            wf = w.astype(np.float64)
            exact = (xf @ wf.T) * s[None, :].astype(np.float64)
            mag = (np.abs(xf) @ np.abs(wf).T) * s[None, :]
            y = _run(fmt, x, w, s).astype(np.float64)
            extra = 0.0
        else:
            wf = O.dequantize_w4(w, s, k).astype(np.float64)
            exact = xf @ wf.T
            mag = np.abs(xf) @ np.abs(wf).T
            y = S.bf16_bits_to_f32(_run(fmt, x, w, s)).astype(np.float64)
            extra = np.abs(exact) * 2.0 ** -8
        gamma = (k + 2) * u / (1 - (k + 2) * u)
        assert np.all(np.abs(y - exact) <= gamma * mag + extra + 1e-30), fmt


# ------------------------------------------------------------ packed layout

def test_nibble_table_exhaustive():
    """All 256 packed bytes: low nibble = even k, two's complement (kernels.c:43-46)."""
    b = np.arange(256, dtype=np.uint8).reshape(256, 1)
    q = O.unpack_i4_rows_to_i8(b, 2)
    lo = np.array([v - 16 if v >= 8 else v for v in range(16)] * 16)
    hi = np.repeat(np.array([v - 16 if v >= 8 else v for v in range(16)]), 16)
    assert np.array_equal(q[:, 0], lo)
    assert np.array_equal(q[:, 1], hi)
    # the oracle's kernels decode the same way: K=2, unit scale, x = (1, 0) and (0, 1)
    ones = np.ones(256, np.float32)
    x = S.f32_to_bf16_bits(np.array([[1, 0], [0, 1]], np.float32))
    y = S.bf16_bits_to_f32(O.linear_w4a16_bf16(x, b, ones))
    assert np.array_equal(y[0], lo.astype(np.float32))
    assert np.array_equal(y[1], hi.astype(np.float32))


@pytest.mark.parametrize("kind", ["i8", "i4row", "i4g32", "i4g128"])
def test_quantizer_invariants(kind):
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((20, 300)) * 0.02).astype(np.float32)
    w[3] = 0.0                                   # an all-zero row -> scale clamps to 1e-8
    w[5, 7] = 0.5                                # an outlier row
    if kind == "i8":
        q, s = O.quantize_weight_i8_per_row(w)
        deq = q.astype(np.float32) * s[:, None]
        qmax, qi = 127, q.astype(np.int64)
        per = s[:, None]
    else:
        if kind == "i4row":
            q, s = O.quantize_weight_i4_per_row(w)
            per = s[:, None]
        else:
            g = 32 if kind == "i4g32" else 128
            q, s = O.quantize_weight_i4_grouped(w, g)
            per = s[:, np.arange(300) // g]
        qi = O.unpack_i4_rows_to_i8(q, 300).astype(np.int64)
        deq = qi.astype(np.float32) * per
        qmax = 7
    assert s.dtype == np.float32 and np.all(s >= np.float32(1e-8))
    assert np.all(np.abs(qi) <= qmax)
    assert np.all(np.abs(deq - w) <= per / 2 * (1 + 1e-6) + 1e-12)
    assert np.all(qi[3] == 0)
    # every non-zero row/group reaches the code +-qmax
    assert np.abs(qi[5]).max() == qmax


def test_quantizer_rounds_half_to_even():
    w = np.array([[7.0, 0.5, 1.5, 2.5, -0.5, -2.5, 3.49]], np.float32)   # max 7 -> scale 1
    q, s = O.quantize_weight_i4_per_row(w)
    assert s[0] == np.float32(1.0)
    assert list(O.unpack_i4_rows_to_i8(q, 7)[0]) == [7, 0, 2, 2, 0, -2, 3]
