"""Pins the oracle's fused epilogues: the elementwise SwiGLU, the fused W4
SwiGLU MLP (kernels.c:1580-1735) and the lm_head argmax's selection rule
(kernels.c:658-737), against the golden vectors written from the reference's
own kernels.c, the reference library built from source (when present),
mathematics (the fp64 SwiGLU, numpy's argmax) and planted mistakes.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from pilm_amd import synth as S
from tests import _golden as GV


def _bits_equal(a, b) -> bool:
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


@pytest.mark.parametrize("case", GV.swiglu_bf16_cases(), ids=lambda c: c["name"])
def test_swiglu_bf16_matches_golden_for_every_gate(case):
    g, u = GV.swiglu_bf16_inputs(case)
    assert GV.sha(g, u) == case["input_sha256"]
    GV.check_output(case, O.swiglu_bf16(g, u))


@pytest.mark.parametrize("case", GV.swiglu_cases(max_weights=1 << 25), ids=lambda c: c["name"])
def test_fused_swiglu_matches_golden(case):
    ins = GV.swiglu_inputs(case)
    assert GV.sha(*ins) == case["input_sha256"]
    GV.check_output(case, O.swiglu_w4a16_bf16(*ins, case["I"]))


def test_fused_swiglu_is_gate_up_linear_then_swiglu_then_down_linear():
    """The fused op equals the composition of three separately pinned ops:
    W4 per-row linear over the 2I gate/up rows, the elementwise SwiGLU of the
    two halves, the W4 per-row linear of the hidden row."""
    gen = GV._gen()
    for t, (h, i, k) in enumerate(((1, 1, 1), (5, 3, 33), (17, 40, 100), (40, 129, 300), (64, 512, 1024))):
        x, gu, gs, dw, ds = gen.make_swiglu_inputs(h, i, k, 31000 + t)
        y, hidden = O.swiglu_w4a16_bf16(x, gu, gs, dw, ds, i, return_hidden=True)
        g_u = O.linear_w4a16_bf16(x, gu, gs)[0]
        h2 = O.swiglu_bf16(g_u[:i], g_u[i:])
        assert _bits_equal(hidden, h2), (h, i, k)
        assert _bits_equal(y, O.linear_w4a16_bf16(h2.reshape(1, -1), dw, ds)), (h, i, k)


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (reference sources absent)")
def test_fused_swiglu_matches_reference_build_fresh_seeds():
    rng = np.random.default_rng(777)
    gen = GV._gen()
    for t in range(40):
        h, i, k = (int(v) for v in (rng.integers(1, 70), rng.integers(1, 300), rng.integers(1, 600)))
        special = (None, "large_gate", "tiny_gate")[t % 3]
        ins = gen.make_swiglu_inputs(h, i, k, 32000 + t, special)
        assert _bits_equal(O.swiglu_w4a16_bf16(*ins, i), O.swiglu_w4a16_bf16(*ins, i, impl="ref")), (h, i, k)
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    for seed in range(3):
        u = np.random.default_rng(seed).integers(0, 65536, 65536).astype(np.uint16)
        assert _bits_equal(O.swiglu_bf16(g, u), O.swiglu_bf16(g, u, impl="ref"))


def test_swiglu_within_half_bf16_ulp_of_fp64():
    """For every finite gate with u = 1 the output is silu(g) (fp64) rounded
    to bf16, to within the fp32 rounding of the intermediate steps."""
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    y = S.bf16_bits_to_f32(O.swiglu_bf16(g, np.full(65536, 0x3F80, np.uint16))).astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        gf = S.bf16_bits_to_f32(g).astype(np.float64)
        exact = gf / (1.0 + np.exp(-gf))
    # Below g = -0x1.62e42ep6 exp(-g) overflows fp32, so 1 + exp(-g) = inf and
    # the fp32 formula gives g / inf = -0 where fp64 still has a tiny value.
    overflow = np.isfinite(gf) & (gf < -88.72283935546875)
    assert np.all(y[overflow] == 0.0) and np.all(np.signbit(y[overflow]))
    fin = np.isfinite(gf) & np.isfinite(exact) & ~overflow
    nonfin = ~np.isfinite(gf)
    assert np.array_equal(np.isnan(y[nonfin]), np.isnan(exact[nonfin]) | np.isnan(gf[nonfin]))
    err = np.abs(y[fin] - exact[fin])
    tiny = np.abs(exact[fin]) < 1e-37          # bf16 subnormal range: absolute bound
    bound = np.where(tiny, 2.0 ** -133, np.abs(exact[fin]) * (2.0 ** -8 + 2.0 ** -20))
    assert np.all(err <= bound)
    assert y[np.where(g == 0)[0][0]] == 0.0                      # silu(0) = 0
    big = fin & (gf > 20)
    assert np.all(y[big] == gf[big])                              # silu(g) = g once exp(-g) < 2^-9 ulp


def test_expf_is_the_c_library_expf():
    x = np.array([0.0, -0.1005859375, 1.0, -88.5, 88.7, -104.0, 89.0], np.float32)
    y = O.expf(x)
    assert y[0] == 1.0 and y[5] == 0.0 and np.isinf(y[6])
    assert np.all(np.abs(y[:5].astype(np.float64) - np.exp(x[:5].astype(np.float64))) <=
                  np.exp(x[:5].astype(np.float64)) * 2.0 ** -23)


PLANTS = {8: "gate/up not rounded to bf16", 9: "expf(g) in silu"}


@pytest.mark.parametrize("variant", sorted(PLANTS), ids=lambda v: PLANTS[v])
def test_golden_vectors_reject_planted_swiglu_mistake(variant):
    for case in GV.swiglu_cases(max_weights=1 << 22):
        y = O.swiglu_w4a16_bf16(*GV.swiglu_inputs(case), case["I"], impl=variant)
        if GV.sha(y) != case["output_sha256"]:
            return
    pytest.fail(f"planted mistake {variant} ({PLANTS[variant]}) passed every golden vector")


def _argmax_rule(v: np.ndarray) -> tuple[int, float]:
    """The reference's scan rule by numpy: NaN never wins, ties and +-0 go to
    the lowest index, (0, -inf) when nothing exceeds -inf."""
    ok = ~np.isnan(v)
    if not ok.any() or v[ok].max() == -np.inf:
        return 0, float("-inf")
    best = v[ok].max()
    idx = int(np.nonzero(ok & (v == best))[0][0])
    return idx, float(v[idx])


def argmax_special_inputs(kind: str, seed: int, n: int = 300, k: int = 64):
    """W8A16 lm_head inputs whose logits hold NaN, +-inf, +-0 or ties."""
    x = S.activations_bf16(seed, 1, k)
    w = S.weights_i8(seed + 1, n, k)
    s = S.scales_uniform(seed + 2, (n,), fp16_round=False)
    rng = np.random.default_rng(seed)
    if kind == "nan_rows":
        s[rng.choice(n, 40, replace=False)] = np.nan
    elif kind == "all_nan":
        s[:] = np.nan
    elif kind == "neg_inf":                       # row 0 NaN (0 * -inf), every other row -inf
        s[:] = -np.inf
        w[:] = 0
        w[1:, 0] = 127
        x[0, 0] = 0x3F80
    elif kind == "pos_inf":
        s[rng.choice(n, 5, replace=False)] = np.inf
    elif kind == "zeros":
        w[:] = 0
        s[::2] = -s[::2]                          # +0 and -0 logits
    elif kind == "ties_late":                     # equal maxima from row n/2 on
        xf = S.bf16_bits_to_f32(x[0])
        w[n // 2:] = (np.sign(xf) * 100).astype(np.int8)
        s[n // 2:] = np.float32(1.0)
    return x, w, s


ARGMAX_KINDS = ("nan_rows", "all_nan", "neg_inf", "pos_inf", "zeros", "ties_late")


@pytest.mark.parametrize("kind", ARGMAX_KINDS)
def test_argmax_rule_on_special_logits(kind):
    x, w, s = argmax_special_inputs(kind, 4100 + ARGMAX_KINDS.index(kind))
    logits = S.bf16_bits_to_f32(O.linear_w8a16_bf16(x, w, s)[0])
    idx, val = O.linear_w8a16_bf16_argmax(x, w, s)
    eidx, evaL = _argmax_rule(logits)
    assert idx == eidx
    assert np.float32(val).tobytes() == np.float32(evaL).tobytes()
    if O.ref_available():
        ridx, rval = O.linear_w8a16_bf16_argmax(x, w, s, impl="ref")
        assert ridx == idx and np.float32(rval).tobytes() == np.float32(val).tobytes()
