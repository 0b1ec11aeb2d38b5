#!/usr/bin/env python3
"""Benchmark of the quantized decode GEMV path on one MI355X.

Workload (one "step"): every W4A16 group-128 linear of one Qwen3-1.7B decode
token, M = 1, in the reference's block layout -- per layer q 4096x2048 (gated
q_proj), k 1024x2048, v 1024x2048, o 2048x2048, gate 6144x2048,
up 6144x2048, down 2048x6144, for 28 layers, plus lm_head 151936x2048.
Every layer has its own weights resident in HBM (0.98 GB per step, far
beyond the 256 MB Infinity Cache), activations are bf16 ~N(0,1), packed int4
weights uniform over all 256 byte values, fp32 group scales ~U(0.001, 0.02)
rounded through fp16.  The step's 197 linear calls go through the C ABI
entry point ekernel_linear_w4a16g128_bf16, captured once into a HIP graph and
replayed.

Printed JSON line:
  value        algorithmic GB/s of the whole step (weights + scales +
               activations + outputs, each counted once) / wall time
  roofline     the g128 GEMV kernel's algorithmic GB/s from per-call HIP
               events on its stream, against the 8 TB/s HBM peak
  cpu_baseline the reference CPU kernel (kernels.c built from source, OpenMP)
               on a bounded sample of the same workload on this host
  sweep        per-shape GB/s at M = 1, 4, 16 (configuration sweep)
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
LAYERS = 28
HIDDEN = 2048
LAYER_SHAPES = [("q_proj", 4096, 2048), ("k_proj", 1024, 2048), ("v_proj", 1024, 2048), ("o_proj", 2048, 2048),
                ("gate_proj", 6144, 2048), ("up_proj", 6144, 2048), ("down_proj", 2048, 6144)]
LM_HEAD = ("lm_head", 151936, 2048)


def alg_bytes(m: int, n: int, k: int) -> int:
    """W4 g128: packed weights + fp32 scales + bf16 activations + bf16 outputs."""
    return n * ((k + 1) // 2) + 4 * n * ((k + 127) // 128) + 2 * m * k + 2 * m * n


def step_shapes():
    return [(name, n, k) for _ in range(LAYERS) for (name, n, k) in LAYER_SHAPES] + [LM_HEAD]


def make_weights(torch, dev, n: int, k: int, gen):
    w = torch.randint(0, 256, (n, (k + 1) // 2), dtype=torch.uint8, device=dev, generator=gen)
    s = (torch.rand((n, (k + 127) // 128), device=dev, generator=gen) * 0.019 + 0.001).half().float()
    return w, s


def build_step(torch, dev, m: int, seed: int = 0):
    """Weights for every call of one step plus fixed inputs/outputs."""
    from pilm_amd import ckernel  # noqa: F401  (loads and checks the library)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    xs = {k: torch.randn((m, k), device=dev, generator=gen).to(torch.bfloat16) for k in (2048, 6144)}
    calls = []
    for name, n, k in step_shapes():
        w, s = make_weights(torch, dev, n, k, gen)
        out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        calls.append((name, n, k, w, s, out))
    return xs, calls


def launcher(torch, xs, calls, m: int):
    """Returns run() issuing every call of the step through the C ABI."""
    from pilm_amd import bindings as abi
    lib = abi._load_lib()
    fn = lib.ekernel_linear_w4a16g128_bf16
    descs = [abi.EkernelLinearW8A32Desc(m, n, k) for (_, n, k, _, _, _) in calls]
    args = [(ctypes.byref(d), ctypes.c_void_p(xs[k].data_ptr()), ctypes.c_void_p(w.data_ptr()),
             ctypes.c_void_p(s.data_ptr()), ctypes.c_void_p(out.data_ptr()), 6)
            for d, (_, n, k, w, s, out) in zip(descs, calls)]

    def run():
        abi.set_stream(torch.cuda.current_stream().cuda_stream)
        for a in args:
            rc = fn(*a)
            if rc != 0:
                raise RuntimeError(f"ekernel_linear_w4a16g128_bf16 failed: rc={rc} ({abi.last_error()})")
    run.keep = (descs, args)
    return run


def capture(torch, run):
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()                      # warm: sizes the split-K scratch before capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, capture_error_mode="relaxed"):
        run()
    torch.cuda.synchronize()
    return g


def time_graph(torch, g, steps: int, warmup: int) -> float:
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g.replay()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def roofline(torch, run, reps: int = 3) -> dict:
    """Per-call HIP event timing of the g128 GEMV (eager launches)."""
    from pilm_amd import bindings as abi
    run()
    torch.cuda.synchronize()
    abi.profile_begin()
    for _ in range(reps):
        run()
    abi.profile_end()
    prof = abi.profile_read()
    fam = prof["w4a16g128_gemv"]
    sec = fam["ms"] / 1e3
    achieved = fam["bytes"] / sec / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "gemv_exact_kernel<W4G128,1> (+ group_fold_kernel when K is split)",
            "calls": fam["calls"], "avg_launch_us": round(fam["ms"] * 1e3 / fam["calls"], 3),
            "alg_bytes_per_launch": round(fam["bytes"] / fam["calls"])}


def sweep(torch, dev, ms=(1, 4, 16), reps: int = 20) -> dict:
    """Per-shape GB/s: each shape replicated across enough copies to bust the
    256 MB Infinity Cache, launched back to back inside one HIP graph."""
    from pilm_amd import bindings as abi
    lib = abi._load_lib()
    fn = lib.ekernel_linear_w4a16g128_bf16
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    res = {}
    shapes = LAYER_SHAPES + [LM_HEAD]
    for name, n, k in shapes:
        per = alg_bytes(1, n, k)
        copies = max(2, min(1024, -(-(512 << 20) // per)))   # >= 512 MB of distinct weights
        ws = [make_weights(torch, dev, n, k, gen) for _ in range(copies)]
        for m in ms:
            x = torch.randn((m, k), device=dev, generator=gen).to(torch.bfloat16)
            out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
            d = abi.EkernelLinearW8A32Desc(m, n, k)

            def run():
                abi.set_stream(torch.cuda.current_stream().cuda_stream)
                for (w, s) in ws:
                    rc = fn(ctypes.byref(d), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(w.data_ptr()),
                            ctypes.c_void_p(s.data_ptr()), ctypes.c_void_p(out.data_ptr()), 6)
                    if rc != 0:
                        raise RuntimeError(abi.last_error())
            g = capture(torch, run)
            sec = time_graph(torch, g, reps, 2)
            calls = reps * copies
            res.setdefault(f"M{m}", {})[name] = {
                "N": n, "K": k, "us": round(sec / calls * 1e6, 2),
                "GBps": round(alg_bytes(m, n, k) * calls / sec / 1e9, 1),
                "TFLOPs": round(2.0 * m * n * k * calls / sec / 1e12, 3)}
            del g
        del ws
        torch.cuda.empty_cache()
    return res


def cpu_baseline(budget_s: float = 12.0) -> dict | None:
    """The reference's ekernel_linear_w4a16g128_bf16 (kernels.c compiled from
    source into oracle/_ref, OpenMP over rows) on this host.  Sample: one
    layer's seven linears plus lm_head at M = 1, repeated for ~budget_s."""
    import numpy as np
    from oracle import oracle as O
    from pilm_amd import synth as S
    kind = "reference" if O.ref_available() else "port"
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    shapes = LAYER_SHAPES + [LM_HEAD]
    data = []
    for i, (name, n, k) in enumerate(shapes):
        x = S.activations_bf16(100 + i, 1, k)
        rng = np.random.default_rng(i)
        w = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
        s = S.scales_uniform(200 + i, (n, k // 128))
        data.append((x, w, s, n, k))
    impl = "ref" if kind == "reference" else "oracle"
    O.linear_w4a16g_bf16(data[0][0], data[0][1], data[0][2], 128, impl=impl)   # warm (OpenMP pool)
    done_bytes, reps = 0, 0
    t0 = time.perf_counter()
    while True:
        for (x, w, s, n, k) in data:
            O.linear_w4a16g_bf16(x, w, s, 128, impl=impl)
            done_bytes += alg_bytes(1, n, k)
        reps += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    sec = time.perf_counter() - t0
    return {"value": round(done_bytes / sec / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": kind,
            "sample": f"{reps} passes over one layer's 7 W4A16-g128 linears + lm_head (M=1) in {sec:.1f} s",
            "cpu": _cpu_model()}


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the decode GEMV would shard by output rows, see DESIGN.md", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    m = 1
    print(f"[bench] building step: {len(step_shapes())} W4A16-g128 linears, M={m}", flush=True)
    xs, calls = build_step(torch, dev, m)
    run = launcher(torch, xs, calls, m)
    step_bytes = sum(alg_bytes(m, n, k) for (_, n, k, *_rest) in calls)
    g = capture(torch, run)
    print(f"[bench] graph captured; timing {args.steps} steps after {args.warmup} warmup", flush=True)
    sec = time_graph(torch, g, args.steps, args.warmup)
    ms_per_step = sec / args.steps * 1e3
    value = step_bytes * args.steps / sec / 1e9

    # eager (no graph) step time, for reference
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        run()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) / 3 * 1e3

    print("[bench] per-call event timing", flush=True)
    roof = roofline(torch, run)
    del g
    out = {
        "metric": "quant GEMV HBM GB/s (% of peak) + Qwen3-1.7B W4A16 decode tok/s, 1 GPU",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights x bf16 activations, fp32 accumulate (bit-exact reference order)",
        "data": "synthetic (seeded torch RNG on device), weights resident in HBM",
        "config": {"workload": "Qwen3-1.7B W4A16-g128 decode linears, one token (28 layers x 7 + lm_head)",
                   "M": m, "calls_per_step": len(calls), "alg_bytes_per_step": step_bytes,
                   "entry_point": "ekernel_linear_w4a16g128_bf16", "launch": "HIP graph replay"},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "decode_linear_tok_s": round(1e3 / ms_per_step, 1),
        "eager_ms_per_step": round(eager_ms, 3),
        "roofline": roof,
    }
    if not args.no_sweep:
        print("[bench] shape sweep M=1,4,16", flush=True)
        del calls, xs, run
        torch.cuda.empty_cache()
        out["sweep"] = sweep(torch, dev)
    if not args.no_cpu:
        print("[bench] cpu baseline", flush=True)
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
