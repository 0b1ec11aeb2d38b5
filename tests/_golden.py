"""Shared access to the committed golden vectors (tests/golden/)."""
from __future__ import annotations

import hashlib
import importlib.util
import json
from functools import lru_cache
from pathlib import Path

import numpy as np

GOLDEN_DIR = Path(__file__).resolve().parent / "golden"


@lru_cache(maxsize=1)
def _gen():
    spec = importlib.util.spec_from_file_location("gen_golden", GOLDEN_DIR / "gen_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@lru_cache(maxsize=1)
def manifest() -> dict:
    return json.loads((GOLDEN_DIR / "linear_golden.json").read_text())


@lru_cache(maxsize=1)
def arrays():
    return dict(np.load(GOLDEN_DIR / "linear_golden.npz", allow_pickle=False))


def linear_cases(max_elems: int | None = None, prefix: str | None = None):
    out = []
    for c in manifest()["cases"]:
        if c["fmt"] in ("w8a16_argmax", "swiglu_w4a16", "swiglu_bf16"):
            continue
        if prefix and not c["name"].startswith(prefix):
            continue
        if max_elems is not None and c["M"] * c["N"] * max(c["K"], 1) > max_elems:
            continue
        out.append(c)
    return out


def argmax_cases():
    return [c for c in manifest()["cases"] if c["fmt"] == "w8a16_argmax"]


def swiglu_cases(max_weights: int | None = None):
    out = [c for c in manifest()["cases"] if c["fmt"] == "swiglu_w4a16"]
    if max_weights is not None:
        out = [c for c in out if c["I"] * (2 * c["K"] + c["N"]) <= max_weights]
    return out


def swiglu_inputs(case: dict):
    """(x, gate_up_qweight, gate_up_scales, down_qweight, down_scales)."""
    return _gen().make_swiglu_inputs(case["N"], case["I"], case["K"], case["seed"], case["special"])


def swiglu_bf16_cases():
    return [c for c in manifest()["cases"] if c["fmt"] == "swiglu_bf16"]


def swiglu_bf16_inputs(case: dict):
    return _gen().swiglu_bf16_inputs(case["special"])


def inputs(case: dict):
    return _gen().make_inputs(case["fmt"], case["M"], case["N"], case["K"], case["seed"], case["special"])


def argmax_inputs(case: dict):
    from pilm_amd import synth as S
    seed, n, k = case["seed"], case["N"], case["K"]
    x = S.activations_bf16(seed, 1, k)
    w = S.weights_i8(seed + 1, n, k)
    s = S.scales_uniform(seed + 2, (n,), fp16_round=False)
    if case["special"] == "ties":
        w[:] = w[0]
        s[:] = s[0]
    return x, w, s


def sha(*arrs) -> str:
    h = hashlib.sha256()
    for a in arrs:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def check_output(case: dict, y: np.ndarray) -> None:
    """Bit-exact comparison of a full output against the golden case."""
    exp = arrays()[case["name"]]
    stride = manifest()["sample_stride"]
    if case["full"]:
        assert y.shape == exp.shape
        y = np.ascontiguousarray(y)
        bad = np.argwhere(y.view(np.uint8) != exp.view(np.uint8))
        assert len(bad) == 0, f"{case['name']}: {len(bad)} mismatching bytes, first at {bad[:3].tolist()}"
    else:
        sample = np.ascontiguousarray(y.reshape(-1)[::stride])
        assert np.array_equal(sample.view(np.uint8), exp.view(np.uint8)), f"{case['name']}: sample mismatch"
    assert sha(y) == case["output_sha256"], f"{case['name']}: output hash mismatch"
