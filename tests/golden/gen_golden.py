"""Write the golden vectors of the quantized linear path and its fused
epilogues (lm_head argmax, W4 SwiGLU MLP, elementwise SwiGLU).

Run in a container that has the piLM sources, after `make -C oracle`:

    python tests/golden/gen_golden.py

Outputs come from the reference's own C kernels (src/ecpu/src/kernel/kernels.c,
compiled from source into oracle/_ref/libecpu_ref.so by oracle/Makefile).
Inputs are regenerated from the recorded seeds by pilm_amd.synth (integer
arithmetic only, so they are identical on every host); a SHA-256 of each
case's inputs is stored so a drift in the generator is caught.

linear_golden.npz holds the full output of every small case; for the large
config shapes it holds a strided sample and linear_golden.json the SHA-256 of
the full output bytes.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle as O  # noqa: E402
from pilm_amd import synth as S  # noqa: E402

OUT = Path(__file__).resolve().parent
FULL_LIMIT = 1 << 15          # outputs up to this many elements are stored whole
SAMPLE_STRIDE = 97

FORMATS = ("w8a32", "w8a16", "w4", "w4g32", "w4g128")


def make_inputs(fmt: str, m: int, n: int, k: int, seed: int, special: str | None = None):
    """Inputs of one case, following the benchmark distributions."""
    if fmt == "w8a32":
        x = S.activations_f32(seed, m, k)
    else:
        x = S.activations_bf16(seed, m, k)
    if fmt.startswith("w8"):
        w = S.weights_i8(seed + 1, n, k)
    else:
        w = S.weights_i4_packed(seed + 1, n, k)
    if fmt in ("w4g32", "w4g128"):
        g = 32 if fmt == "w4g32" else 128
        s = S.scales_uniform(seed + 2, (n, (k + g - 1) // g))
    else:
        s = S.scales_uniform(seed + 2, (n,), fp16_round=False)
    if special == "zero_x":
        x = np.zeros_like(x)
    elif special == "min_w":                      # every weight at its most negative code
        w = np.full_like(w, -128 if fmt.startswith("w8") else 0x88)
    elif special == "denormal_x":                 # subnormal fp32 / bf16 activations
        if fmt == "w8a32":
            x = (x * np.float32(1e-39)).astype(np.float32)
        else:
            x = S.f32_to_bf16_bits(S.bf16_bits_to_f32(x) * np.float32(1e-39))
    elif special == "large_x":                    # near the top of the fp32 range
        if fmt == "w8a32":
            x = (x * np.float32(1e30)).astype(np.float32)
        else:
            x = S.f32_to_bf16_bits(S.bf16_bits_to_f32(x) * np.float32(1e30))
    elif special in ("cancel_halves", "cancel_groups"):
        # Exact cancellation makes the result equal to a rounding error of the
        # reference's own operation order, so an output that survives bf16
        # rounding depends on that order (FMA vs separate roundings, one
        # accumulator vs the lo/hi halves).
        span = 8 if special == "cancel_halves" else (32 if fmt == "w4g32" else 128)
        xf = x.astype(np.float32) if fmt == "w8a32" else S.bf16_bits_to_f32(x)
        xf = xf.copy()
        for k0 in range(0, k - 2 * span + 1, 2 * span):
            xf[:, k0 + span:k0 + 2 * span] = -xf[:, k0:k0 + span]
        x = xf if fmt == "w8a32" else S.f32_to_bf16_bits(xf)
        if fmt.startswith("w8"):
            for k0 in range(0, k - 2 * span + 1, 2 * span):
                w[:, k0 + span:k0 + 2 * span] = w[:, k0:k0 + span]
        else:
            b = span // 2
            for j0 in range(0, (k // 2) - 2 * b + 1, 2 * b):
                w[:, j0 + b:j0 + 2 * b] = w[:, j0:j0 + b]
        if s.ndim == 2:
            s[:, 1::2] = s[:, 0::2][:, :s[:, 1::2].shape[1]]
    return x, w, s


def run(fmt: str, x, w, s, impl: str):
    if fmt == "w8a32":
        return O.linear_w8a32(x, w, s, impl=impl)
    if fmt == "w8a16":
        return O.linear_w8a16_bf16(x, w, s, impl=impl)
    if fmt == "w4":
        return O.linear_w4a16_bf16(x, w, s, impl=impl)
    return O.linear_w4a16g_bf16(x, w, s, 32 if fmt == "w4g32" else 128, impl=impl)


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def cases():
    """(name, fmt, M, N, K, seed, special)"""
    out = []
    seed = 1000
    for fmt in FORMATS:
        for k in (1, 2, 7, 8, 15, 16, 17, 127, 128, 129, 256):
            for n in (1, 7, 8, 9, 17):
                for m in (1, 2, 5):
                    seed += 7
                    out.append((f"{fmt}_M{m}_N{n}_K{k}", fmt, m, n, k, seed, None))
        # stripe-aligned K with ragged N (partial 64-row tiles on the GPU)
        for (m, n, k) in ((1, 100, 256), (3, 65, 384), (5, 130, 1024), (2, 1, 512), (4, 63, 640)):
            seed += 7
            out.append((f"{fmt}_M{m}_N{n}_K{k}", fmt, m, n, k, seed, None))
        for special in ("zero_x", "min_w", "denormal_x", "large_x"):
            seed += 7
            out.append((f"{fmt}_{special}", fmt, 2, 70, 256, seed, special))
        for special in ("cancel_halves", "cancel_groups"):
            for (m, n, k) in ((1, 200, 512), (3, 64, 2048)):
                seed += 7
                out.append((f"{fmt}_{special}_M{m}_N{n}_K{k}", fmt, m, n, k, seed, special))
    # configuration 1: W8A32 GEMV, x fp32 [1,4096], W int8 [4096,4096]
    out.append(("config1_w8a32_M1_N4096_K4096", "w8a32", 1, 4096, 4096, 1, None))
    # configuration 2: Qwen3-1.7B projections (gated q 4096, std q/o 2048, k/v 1024,
    # gate/up 6144, fused gate_up 12288, down 2048x6144, lm_head 151936), M in {1,4,16}
    shapes = [(4096, 2048), (2048, 2048), (1024, 2048), (6144, 2048), (12288, 2048), (2048, 6144),
              (151936, 2048)]
    for fmt in ("w4g128", "w4"):
        for (n, k) in shapes:
            for m in (1, 4, 16):
                out.append((f"config2_{fmt}_M{m}_N{n}_K{k}", fmt, m, n, k, 2000 + n + k + m, None))
    return out


def argmax_cases():
    res = []
    for i, (n, k) in enumerate(((1, 8), (7, 9), (17, 256), (1000, 1024), (4096, 2048))):
        res.append((f"argmax_N{n}_K{k}", n, k, 5000 + i))
    # ties: identical rows -> lowest index wins
    res.append(("argmax_ties", 64, 128, 5100))
    return res


def swiglu_cases():
    """(name, H, I, K, seed, special) of the fused W4 SwiGLU (M = 1)."""
    res = []
    seed = 7000
    for (h, i, k) in ((1, 1, 1), (7, 9, 17), (16, 24, 64), (33, 70, 129), (64, 100, 256), (130, 257, 513),
                      (96, 256, 512), (200, 1000, 768), (64, 264, 256)):
        seed += 11
        res.append((f"swiglu_w4_H{h}_I{i}_K{k}", h, i, k, seed, None))
    for special in ("large_gate", "tiny_gate"):
        seed += 11
        res.append((f"swiglu_w4_{special}", 64, 512, 256, seed, special))
    # the MLP of the two decode configurations: Qwen3-1.7B and Qwen3-8B
    res.append(("swiglu_w4_qwen3_1p7b", 2048, 6144, 2048, 7500, None))
    res.append(("swiglu_w4_qwen3_8b", 4096, 12288, 4096, 7501, None))
    return res


def make_swiglu_inputs(h: int, i: int, k: int, seed: int, special: str | None = None):
    x = S.activations_bf16(seed, 1, k)
    gu = S.weights_i4_packed(seed + 1, 2 * i, k)
    gs = S.scales_uniform(seed + 2, (2 * i,), fp16_round=False)
    dw = S.weights_i4_packed(seed + 3, h, i)
    ds = S.scales_uniform(seed + 4, (h,), fp16_round=False)
    if special == "large_gate":       # |g| up to ~1e3: expf overflows / underflows, silu saturates
        gs = (gs * np.float32(300.0)).astype(np.float32)
    elif special == "tiny_gate":      # |g| ~ 1e-6: silu(g) ~ g / 2
        gs = (gs * np.float32(1e-6)).astype(np.float32)
    return x, gu, gs, dw, ds


def swiglu_bf16_inputs(which: str):
    """Every bf16 bit pattern as the gate, against u = 1.0 or seeded u bits."""
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    if which == "u_one":
        u = np.full(65536, 0x3F80, np.uint16)
    else:
        u = S.activations_bf16(7900, 1, 65536).reshape(-1)
    return g, u


def main() -> int:
    if not O.ref_available():
        O.build(ref=True)
    arrays = {}
    manifest = {"generator": "tests/golden/gen_golden.py", "source": "reference kernels.c via oracle/_ref",
                "sample_stride": SAMPLE_STRIDE, "cases": []}
    for (name, fmt, m, n, k, seed, special) in cases():
        x, w, s = make_inputs(fmt, m, n, k, seed, special)
        y = run(fmt, x, w, s, "ref")
        entry = {"name": name, "fmt": fmt, "M": m, "N": n, "K": k, "seed": seed, "special": special,
                 "input_sha256": sha(x, w, s), "output_sha256": sha(y), "full": bool(y.size <= FULL_LIMIT)}
        arrays[name] = y if y.size <= FULL_LIMIT else y.reshape(-1)[::SAMPLE_STRIDE].copy()
        manifest["cases"].append(entry)
    for (name, n, k, seed) in argmax_cases():
        x = S.activations_bf16(seed, 1, k)
        w = S.weights_i8(seed + 1, n, k)
        if name == "argmax_ties":
            w[:] = w[0]
        s = S.scales_uniform(seed + 2, (n,), fp16_round=False)
        if name == "argmax_ties":
            s[:] = s[0]
        idx, val = O.linear_w8a16_bf16_argmax(x, w, s, impl="ref")
        manifest["cases"].append({"name": name, "fmt": "w8a16_argmax", "M": 1, "N": n, "K": k, "seed": seed,
                                  "special": "ties" if name == "argmax_ties" else None,
                                  "input_sha256": sha(x, w, s), "index": idx, "value": val})
    for (name, h, i, k, seed, special) in swiglu_cases():
        ins = make_swiglu_inputs(h, i, k, seed, special)
        y = O.swiglu_w4a16_bf16(*ins, i, impl="ref")
        arrays[name] = y
        manifest["cases"].append({"name": name, "fmt": "swiglu_w4a16", "M": 1, "N": h, "K": k, "I": i,
                                  "seed": seed, "special": special, "input_sha256": sha(*ins),
                                  "output_sha256": sha(y), "full": True})
    for which in ("u_one", "u_seeded"):
        g, u = swiglu_bf16_inputs(which)
        y = O.swiglu_bf16(g, u, impl="ref")
        name = f"swiglu_bf16_all_gates_{which}"
        arrays[name] = y
        manifest["cases"].append({"name": name, "fmt": "swiglu_bf16", "M": 1, "N": 65536, "K": 0, "seed": 7900,
                                  "special": which, "input_sha256": sha(g, u), "output_sha256": sha(y),
                                  "full": True})
    np.savez_compressed(OUT / "linear_golden.npz", **arrays)
    (OUT / "linear_golden.json").write_text(json.dumps(manifest, indent=1) + "\n")
    print(f"wrote {len(manifest['cases'])} cases")
    return 0


if __name__ == "__main__":
    sys.exit(main())
