#!/usr/bin/env python3
"""Benchmark of the quantized decode GEMV path on one MI355X.

Workload (one "step"): every W4A16 group-128 linear of one Qwen3-1.7B decode
token, M = 1, in the reference's block layout, as the device decoder
(pilm_amd.qwen3) issues them -- per layer the q/k/v projections as one
6144x2048 matrix (gated q 4096 + k 1024 + v 1024 rows), o 2048x2048, gate/up
as one 12288x2048 matrix, down 2048x6144, for 28 layers, plus lm_head
151936x2048 (113 calls; --layout separate issues the 197 per-projection
calls instead; the bytes are the same).  Every layer has its own weights
resident in HBM (0.98 GB per step, far beyond the 256 MB Infinity Cache),
activations are bf16 ~N(0,1), packed int4 weights uniform over all 256 byte
values, fp32 group scales ~U(0.001, 0.02) rounded through fp16.  The calls go
through the C ABI entry point ekernel_linear_w4a16g128_bf16, captured once
into a HIP graph and replayed.

Then the whole decoder (--no-decode skips it): Qwen3-1.7B W4A16-g128 with
random-init weights (seed 1, generated and quantized on the device), a
128-token prompt prefilled in 16-token chunks, 256 greedy tokens with the
decode step replayed as one HIP graph; decode tok/s over the 255 graph steps,
and whether the tokens equal the reference engine's
(tests/golden/decode_qwen3_1p7b.json).

Printed JSON line:
  value        algorithmic GB/s of the whole step (weights + scales +
               activations + outputs, each counted once) / wall time
  hbm_copy_GBps  a 1 GiB device copy timed the same way (read + write), the
               attainable streaming rate; pct_of_copy_peak = value against it
  roofline     the g128 GEMV kernels' algorithmic GB/s per launch (the
               group-quad kernels for qkv (16-row tiles) and o/down (8-row
               tiles), the 64-row exact kernel for gate_up and lm_head; they
               are the step's only kernels): HIP events on the replay stream
               around the timed replays, divided by the launches, against
               8 TB/s
  decode_tok_s whole-decoder greedy tokens per second (attention, norms, rope,
               SwiGLU, lm_head and argmax included), HIP graph per token
  cpu_baseline the reference CPU kernel (kernels.c built from source, OpenMP)
               on a bounded sample of the same workload on this host
  sweep        per-shape times with --sweep [sections]: g128 (default),
               w4row, w8a32, w8a16, gemm, gemm_fp16 (torch's fp16 GEMM at
               the same shapes, for reference), fused, attention, load
               (bundle -> HBM), verify (16-sequence MTP verify, M = 80),
               verify_step (the whole batched verify step, Qwen3-1.7B W4A16
               g128), verify_step_8b (the same on Qwen3-8B with int8
               per-row weights, 256-token prompts), or all

Profiling helpers (rocprofv3 runs the program, these read its output):
  --pmc-pass            eager steps plus a plain copy kernel of known size,
                        for one rocprofv3 --pmc counter pass
  --traffic F W         FETCH_SIZE / WRITE_SIZE counter CSVs of two such
                        passes -> HBM bytes per GEMV launch, calibrated by
                        the copy kernel; written to profiles/ and reported as
                        roofline.traffic while the kernel source is unchanged
  --stats-summary CSV   rocprofv3 --kernel-trace --stats output -> summary
  --attn-pmc-pass       paged-attention calls (Qwen3-8B heads, one decode row,
                        32768 positions) plus the copy kernel, for one
                        counter pass
  --attn-traffic F W    FETCH_SIZE / WRITE_SIZE CSVs of two such passes ->
                        bytes per dispatch of each attention kernel beside
                        the K or V bytes it must read
  --shape-pmc-pass      the Qwen3-8B GEMV shapes (W4A16 g128 and W8A32, M=1),
                        the 80-row exact verify and three matrix-core GEMMs,
                        each --steps times after a marker kernel, then the
                        copy kernel, for one counter pass
  --shape-counters S F  the SQ/GRBM and FETCH_SIZE CSVs of two such passes
                        -> per-shape table (time, HBM bytes vs algorithmic,
                        wait share, VALU and MFMA busy, VALU per MFMA)
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
KERNEL_SRCS = [ROOT / "pilm_amd" / "csrc" / f for f in ("linear_exact.hip", "linear_rows.hip", "gemv_device.h")]
# The kernels of the W4A16 group-128 GEMV path at M=1: the group-quad kernel
# for the projections (8-row tiles below 4096 rows, 16-row tiles up to 8192),
# the 64-row exact kernel for lm_head.
GEMV_KERNELS = ("gemv_gq_kernel<3, 1,", "gemv_gq8_kernel<3,", "gemv_exact_kernel<3, 1>")
GEMV_KERNEL = "gemv_gq_kernel<3, 1, *> + gemv_gq8_kernel<3, *> + gemv_exact_kernel<3, 1>"
TRAFFIC_FILE = ROOT / "profiles" / "gemv_w4a16g128_m1_qwen3_1p7b_decode.traffic.txt"
CALIB_BYTES = 1 << 30                              # copy kernel: reads and writes 1 GiB
LAYERS = 28
HIDDEN = 2048
LAYER_SHAPES_SEPARATE = [("q_proj", 4096, 2048), ("k_proj", 1024, 2048), ("v_proj", 1024, 2048),
                         ("o_proj", 2048, 2048), ("gate_proj", 6144, 2048), ("up_proj", 6144, 2048),
                         ("down_proj", 2048, 6144)]
LAYER_SHAPES_FUSED = [("qkv_proj", 6144, 2048), ("o_proj", 2048, 2048), ("gate_up_proj", 12288, 2048),
                      ("down_proj", 2048, 6144)]
LAYER_SHAPES = LAYER_SHAPES_FUSED
LM_HEAD = ("lm_head", 151936, 2048)


def alg_bytes(m: int, n: int, k: int) -> int:
    """W4 g128: packed weights + fp32 scales + bf16 activations + bf16 outputs."""
    return n * ((k + 1) // 2) + 4 * n * ((k + 127) // 128) + 2 * m * k + 2 * m * n


def step_shapes():
    return [(name, n, k) for _ in range(LAYERS) for (name, n, k) in LAYER_SHAPES] + [LM_HEAD]


def decode_bench(torch, dev, n_new: int = 256, prompt_len: int = 128, seed: int = 1) -> dict:
    """The device decoder on Qwen3-1.7B W4A16-g128: prefill, then n_new - 1
    graph-replayed decode steps timed between HIP events on the replay stream
    (wall clock beside them)."""
    from pilm_amd import qwen3 as Q
    from pilm_amd import synth_model as SM
    cfg = Q.QWEN3_1P7B
    t0 = time.perf_counter()
    w = Q.Qwen3Weights.synthetic(cfg, seed, 0.02, device=dev)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    dec = Q.Qwen3Decoder(w, max_positions=prompt_len + n_new + 1, max_new_tokens=n_new)
    prompt = SM.token_ids(seed, prompt_len, cfg.vocab).tolist()
    dec.prefill(prompt)
    dec.capture()
    s = torch.cuda.current_stream(dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dec.prefill(prompt)
    torch.cuda.synchronize()
    prefill_ms = (time.perf_counter() - t0) * 1e3
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(s)
    for _ in range(n_new - 1):
        dec.graph.replay()
    e1.record(s)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu = e0.elapsed_time(e1) / 1e3
    tokens = dec.tokens[:n_new].tolist()
    fx_path = ROOT / "tests" / "golden" / "decode_qwen3_1p7b.json"
    match = None
    if fx_path.exists():
        fx = json.loads(fx_path.read_text())
        if fx["prompt"] == prompt and fx["config"]["seed"] == seed:
            match = tokens == fx["tokens"][:n_new]
    steps = n_new - 1
    return {"decode_tok_s": round(steps / wall, 1), "ms_per_token": round(wall / steps * 1e3, 4),
            "gpu_ms_per_token": round(gpu / steps * 1e3, 4), "prefill_ms": round(prefill_ms, 2),
            "prompt_tokens": prompt_len, "new_tokens": n_new, "tokens_match_reference": match,
            "linear_bytes_per_token": w.linear_bytes_per_token(), "weights_build_s": round(build_s, 2),
            "launch": "one HIP graph per decode token (state word advanced on device)"}


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


def time_graph(torch, g, steps: int, warmup: int, events: bool = False):
    """Wall seconds for `steps` replays; with events=True also the GPU
    seconds between HIP events recorded on the replay stream around them."""
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return (wall, e0.elapsed_time(e1) / 1e3) if events else wall


def roofline(gpu_sec: float, launches: int, bytes_per_launch: float) -> dict:
    """The g128 GEMV kernels are the only kernels of the step: their average
    launch duration is the HIP-event time of the timed replays over the
    launches."""
    avg = gpu_sec / launches
    achieved = bytes_per_launch / avg / 1e9
    traffic, traffic_note = measured_traffic()
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": GEMV_KERNEL + " (K divided among waves, folded inside the kernel)",
            "launches": launches, "avg_launch_us": round(avg * 1e6, 3),
            "alg_bytes_per_launch": round(bytes_per_launch), "traffic_source": traffic_note}


def source_hash() -> str:
    import hashlib
    h = hashlib.sha256()
    for f in KERNEL_SRCS:
        h.update(f.read_bytes())
    return h.hexdigest()


def measured_traffic():
    """HBM bytes per launch from the committed counter summary, if it was
    measured on the current kernel source; (None, reason) otherwise."""
    try:
        rec = json.loads(TRAFFIC_FILE.read_text().strip().splitlines()[-1])
    except (OSError, ValueError, IndexError):
        return None, "no counter summary"
    if rec.get("source_sha256") != source_hash():
        return None, "counter summary is for another kernel source"
    return rec["traffic"], TRAFFIC_FILE.name


def _fmt_bytes(fmt: str, m: int, n: int, k: int) -> int:
    """Algorithmic bytes of one call: weights + scales + activations + outputs."""
    if fmt == "w8a32":
        return n * k + 4 * n + 4 * m * k + 4 * m * n
    if fmt == "w8a16":
        return n * k + 4 * n + 2 * m * k + 2 * m * n
    if fmt == "w4row":
        return n * ((k + 1) // 2) + 4 * n + 2 * m * k + 2 * m * n
    return alg_bytes(m, n, k)   # w4g128


def _fmt_weights(torch, dev, fmt: str, n: int, k: int, gen):
    if fmt in ("w8a32", "w8a16"):
        w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev, generator=gen)
        return w, torch.rand((n,), device=dev, generator=gen) * 0.019 + 0.001
    if fmt == "w4row":
        w = torch.randint(0, 256, (n, (k + 1) // 2), dtype=torch.uint8, device=dev, generator=gen)
        return w, (torch.rand((n,), device=dev, generator=gen) * 0.019 + 0.001).half().float()
    return make_weights(torch, dev, n, k, gen)


_ENTRY = {"w8a32": "ekernel_linear_w8a32", "w8a16": "ekernel_linear_w8a16_bf16",
          "w4row": "ekernel_linear_w4a16_bf16", "w4g128": "ekernel_linear_w4a16g128_bf16"}


def time_linear(torch, dev, fmt: str, n: int, k: int, ms, reps: int = 20, min_bytes: int = 512 << 20) -> dict:
    """One shape of one format at each M: enough distinct weight copies to
    bust the 256 MB Infinity Cache, launched back to back in one HIP graph."""
    from pilm_amd import bindings as abi
    lib = abi._load_lib()
    fn = getattr(lib, _ENTRY[fmt])
    gen = torch.Generator(device=dev)
    gen.manual_seed(n * 7 + k)
    copies = max(2, min(1024, -(-min_bytes // _fmt_bytes(fmt, 1, n, k))))
    ws = [_fmt_weights(torch, dev, fmt, n, k, gen) for _ in range(copies)]
    res = {}
    for m in ms:
        x = torch.randn((m, k), device=dev, generator=gen)
        x = x if fmt == "w8a32" else x.to(torch.bfloat16)
        out = torch.empty((m, n), dtype=torch.float32 if fmt == "w8a32" else torch.bfloat16, device=dev)
        d = abi.EkernelLinearW8A32Desc(m, n, k)

        def run():
            abi.set_stream(torch.cuda.current_stream().cuda_stream)
            for (w, sc) in ws:
                rc = fn(ctypes.byref(d), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(w.data_ptr()),
                        ctypes.c_void_p(sc.data_ptr()), ctypes.c_void_p(out.data_ptr()), 6)
                if rc != 0:
                    raise RuntimeError(abi.last_error())
        g = capture(torch, run)
        sec = time_graph(torch, g, reps, 2)
        calls = reps * copies
        res[f"M{m}"] = {"us": round(sec / calls * 1e6, 2),
                        "GBps": round(_fmt_bytes(fmt, m, n, k) * calls / sec / 1e9, 1),
                        "TFLOPs": round(2.0 * m * n * k * calls / sec / 1e12, 2)}
        del g
    del ws
    torch.cuda.empty_cache()
    return res


# 1.7B projections (per-row W4 uses the fused gate_up shape, as the
# reference's SwiGLU fusion does), 8B projections (gated q, fused gate_up).
SHAPES_1P7B_ROW = [("q_proj", 4096, 2048), ("k_proj", 1024, 2048), ("o_proj", 2048, 2048),
                   ("gate_up_proj", 12288, 2048), ("down_proj", 2048, 6144), LM_HEAD]
SHAPES_8B = [("q_proj", 8192, 4096), ("k_proj", 1024, 4096), ("o_proj", 4096, 4096),
             ("gate_up_proj", 24576, 4096), ("down_proj", 4096, 12288), ("lm_head", 151936, 4096)]


def copy_peak(torch, dev, nbytes: int = 1 << 30, reps: int = 10) -> float:
    """Measured device-copy bandwidth on this GPU (read + write of a 1 GiB
    tensor, HIP graph replay): the attainable streaming rate that the
    datasheet's 8 TB/s overstates."""
    src = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    g = capture(torch, lambda: [dst.copy_(src) for _ in range(reps)])
    sec = time_graph(torch, g, 3, 1)
    del g, src, dst
    torch.cuda.empty_cache()
    return 2 * nbytes * reps * 3 / sec / 1e9


def sweep(torch, dev, sections) -> dict:
    """Per-shape times of the measurement configurations:
      g128   W4A16 g128 at the Qwen3-1.7B shapes, M = 1, 4, 16, and the 8B shapes, M = 1
      w4row  per-row W4A16 (bundle v2) at the 1.7B shapes, M = 1, 4, 16
      w8a32  W8A32: 4096x4096 (the single-GEMV configuration) and the 8B shapes, M = 1
      w8a16  W8A16 at the 8B shapes, M = 1 and 5 (MTP verify of one sequence)
      gemm   prefill / verify at the 8B shapes, W8A32, W8A16 and W4A16 g128,
             M = 64, 256, 1024, 2048 (matrix cores; TFLOP/s)
      fused  W4 SwiGLU MLP and W8A16 lm_head argmax vs their unfused calls
      attention  paged attention of one sequence (decode and MTP verify) at
             the 1.7B and 8B head layouts, 384 .. 131072 positions (K+V GB/s)
      load   a 1.7B W4 bundle uploaded to HBM (GB/s)
      verify MTP verify of 16 sequences x (1 + 4 drafts) at the 8B shapes,
             W8A16 and W4A16 g128: one M = 80 call on the exact kernels,
             the same on the matrix cores, and 16 per-sequence M = 5 calls."""
    res = {}
    if "g128" in sections:
        res["g128_1p7b"] = {name: {"N": n, "K": k, **time_linear(torch, dev, "w4g128", n, k, (1, 4, 16))}
                            for name, n, k in LAYER_SHAPES + [LM_HEAD]}
        res["g128_8b"] = {name: {"N": n, "K": k, **time_linear(torch, dev, "w4g128", n, k, (1,))}
                          for name, n, k in SHAPES_8B}
    if "w4row" in sections:
        res["w4row_1p7b"] = {name: {"N": n, "K": k, **time_linear(torch, dev, "w4row", n, k, (1, 4, 16))}
                             for name, n, k in SHAPES_1P7B_ROW}
    if "w8a32" in sections:
        res["w8a32"] = {name: {"N": n, "K": k, **time_linear(torch, dev, "w8a32", n, k, (1,))}
                        for name, n, k in [("single_4096x4096", 4096, 4096)] + SHAPES_8B}
    if "w8a16" in sections:
        res["w8a16_8b"] = {name: {"N": n, "K": k, **time_linear(torch, dev, "w8a16", n, k, (1, 5))}
                           for name, n, k in SHAPES_8B}
    if "gemm" in sections:
        gm = (64, 256, 1024, 2048)
        res["gemm_8b"] = {f"{fmt}_{name}": {"N": n, "K": k, **time_linear(torch, dev, fmt, n, k, gm, reps=5,
                                                                         min_bytes=256 << 20)}
                          for fmt in ("w8a32", "w8a16", "w4g128") for name, n, k in SHAPES_8B if name != "lm_head"}
    if "gemm_fp16" in sections:
        res["gemm_fp16_8b"] = sweep_gemm_fp16(torch, dev, (64, 256, 1024, 2048))
    if "fused" in sections:
        res["fused"] = sweep_fused(torch, dev)
    if "attention" in sections:
        res["attention"] = sweep_attention(torch, dev)
    if "load" in sections:
        res["load"] = sweep_load(torch, dev)
    if "verify" in sections:
        res["verify_8b"] = sweep_verify(torch, dev)
    if "verify_step" in sections:
        res["verify_step_1p7b"] = sweep_verify_step(torch, dev)
    if "verify_step_8b" in sections:
        from pilm_amd import qwen3 as Q
        res["verify_step_8b_w8"] = sweep_verify_step(torch, dev, cfg=Q.QWEN3_8B_W8, prompt_len=256)
    return res


def sweep_gemm_fp16(torch, dev, ms, reps: int = 20) -> dict:
    """The plain fp16 GEMM of torch (hipBLASLt) at the 8B shapes, fp16
    weights already in HBM: what the matrix cores reach without a weight
    decode, as a reference for the quantized GEMMs (TFLOP/s = 2MNK / time)."""
    res = {}
    for name, n, k in SHAPES_8B:
        if name == "lm_head":
            continue
        w = torch.randn((n, k), device=dev, dtype=torch.float16)
        row = {"N": n, "K": k}
        for m in ms:
            a = torch.randn((m, k), device=dev, dtype=torch.float16)
            for _ in range(3):
                torch.matmul(a, w.t())
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            for _ in range(reps):
                torch.matmul(a, w.t())
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / reps
            row[f"M{m}"] = {"us": round(us, 2), "TFLOPs": round(2.0 * m * n * k / us / 1e6, 1)}
        res[name] = row
        del w
    return res


def sweep_verify_step(torch, dev, n_seq: int = 16, drafts: int = 4, steps: int = 8, prompt_len: int = 128,
                      seed: int = 1, cfg=None) -> dict:
    """One batched MTP verify step end to end, on Qwen3-1.7B W4A16-g128 unless
    cfg names another model (Qwen3Batch.verify: n_seq sequences x (1 +
    drafts) rows through every linear as one M, rope and attention for all
    sequences in one launch each, lm_head on every row, acceptance on the
    host): GPU time between HIP events and wall time per step after a
    prefill of every prompt, with the linears on the bit-exact kernels
    ("exact") and with batches of 64 rows or more on the matrix cores
    ("matrix_cores", within their tolerance).  The drafts are fixed tokens
    (mostly rejected): the step's work is the same whatever is accepted,
    every row goes through the model."""
    from pilm_amd import qwen3 as Q
    from pilm_amd import synth_model as SM
    cfg = cfg or Q.QWEN3_1P7B
    t_w = time.perf_counter()
    w = Q.Qwen3Weights.synthetic(cfg, seed, 0.02, device=dev)
    torch.cuda.synchronize()
    t_w = time.perf_counter() - t_w
    prompts = [SM.token_ids(seed + i, prompt_len, cfg.vocab).tolist() for i in range(n_seq)]
    m = n_seq * (1 + drafts)
    res = {"model": f"Qwen3 {cfg.layers} layers, hidden {cfg.hidden}, {cfg.weights}", "sequences": n_seq,
           "prompt_tokens": prompt_len, "rows_per_step": m, "steps": steps, "weights_build_s": round(t_w, 2)}
    for mode, exact in (("exact", True), ("matrix_cores", False)):
        b = Q.Qwen3Batch(w, n_seqs=n_seq, max_positions=prompt_len + (steps + 2) * (1 + drafts) + 1,
                         max_rows=m, exact=exact)
        torch.cuda.synchronize()
        t_p = time.perf_counter()
        last = b.prefill_seqs(list(range(n_seq)), prompts)
        torch.cuda.synchronize()
        t_p = time.perf_counter() - t_p
        drafts_of = [[0] * drafts for _ in range(n_seq)]
        s = torch.cuda.current_stream(dev)
        gpu_ms, wall_ms, accepted = [], [], 0
        for it in range(steps + 1):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            e0.record(s)
            out = b.verify(last, drafts_of)
            e1.record(s)
            torch.cuda.synchronize()
            if it > 0:                                     # the first step warms the descriptors and scratch
                wall_ms.append((time.perf_counter() - t0) * 1e3)
                gpu_ms.append(e0.elapsed_time(e1))
                accepted += sum(len(a) for a, _ in out)
            last = [nxt for _, nxt in out]
        g = sorted(gpu_ms)[len(gpu_ms) // 2]
        res[mode] = {"gpu_ms_per_step": round(g, 3), "wall_ms_per_step": round(sorted(wall_ms)[len(wall_ms) // 2], 3),
                     "rows_per_s": round(m / g * 1e3, 1), "accepted_drafts_per_step": round(accepted / steps, 1),
                     # a step emits n_seq tokens plus the accepted drafts: no draft / every draft accepted
                     "tokens_per_s_bounds": [round(n_seq / g * 1e3, 1), round(m / g * 1e3, 1)],
                     "prefill_s": round(t_p, 2)}
        del b
        torch.cuda.empty_cache()
    return res


def sweep_verify(torch, dev, n_seq: int = 16, drafts: int = 4) -> dict:
    """Batched MTP verify: M = n_seq * (1 + drafts) rows per linear."""
    from pilm_amd import bindings as abi
    m1 = 1 + drafts
    m = n_seq * m1
    res = {}
    for fmt in ("w8a16", "w4g128"):
        for name, n, k in SHAPES_8B:
            prev = abi.matrix_core_min_rows()
            abi.set_matrix_core_min_rows(0)
            try:
                exact = time_linear(torch, dev, fmt, n, k, (m1, m), reps=5, min_bytes=256 << 20)
            finally:
                abi.set_matrix_core_min_rows(prev)
            mc = time_linear(torch, dev, fmt, n, k, (m,), reps=5, min_bytes=256 << 20)
            res[f"{fmt}_{name}"] = {"N": n, "K": k,
                                    f"exact_M{m}_us": exact[f"M{m}"]["us"],
                                    f"matrix_M{m}_us": mc[f"M{m}"]["us"],
                                    f"per_seq_{n_seq}xM{m1}_us": round(n_seq * exact[f"M{m1}"]["us"], 2),
                                    f"exact_M{m}_GBps": exact[f"M{m}"]["GBps"]}
            print(f"[bench] verify {fmt} {name}: {res[f'{fmt}_{name}']}", file=sys.stderr, flush=True)
    return res


def sweep_load(torch, dev) -> dict:
    """Bundle upload: a synthetic Qwen3-1.7B W4A16 per-row bundle (28 layers x
    7 linears + lm_head, export_pilm_quant_bundle_v2 layout) written to a
    temporary directory, then loaded into one HBM arena by pilm_amd.weights
    (file -> pinned staging -> HBM).  The files were just written, so they
    are read from the page cache: the rate is host memory -> HBM, not disk."""
    import shutil
    import tempfile

    import numpy as np

    from pilm_amd import weights as Wt
    rng = np.random.default_rng(5)
    lin = {}
    for layer in range(LAYERS):
        for name, n, k in LAYER_SHAPES:
            lin[f"model.layers.{layer}.{name}.weight"] = (
                torch.from_numpy(rng.integers(0, 256, (n, (k + 1) // 2), dtype=np.uint8)),
                torch.from_numpy((rng.random(n, dtype=np.float32) * 0.019 + 0.001)), k)
    lin["lm_head.weight"] = (torch.from_numpy(rng.integers(0, 256, (LM_HEAD[1], LM_HEAD[2] // 2), dtype=np.uint8)),
                             torch.from_numpy(rng.random(LM_HEAD[1], dtype=np.float32)), LM_HEAD[2])
    tmp = tempfile.mkdtemp(prefix="pilm_bundle_")
    try:
        t0 = time.perf_counter()
        Wt.write_bundle(tmp, "w4a16", lin)
        write_s = time.perf_counter() - t0
        runs = []
        for _ in range(2):
            b = Wt.QuantBundle(tmp, dev)
            torch.cuda.synchronize()
            runs.append(b.stats)
            del b
            torch.cuda.empty_cache()
        best = max(runs, key=lambda r: r["GBps"])
        return {"linears": best["linears"], "bytes": best["bytes"], "seconds": round(best["seconds"], 3),
                "GBps": round(best["GBps"], 2), "runs_GBps": [round(r["GBps"], 2) for r in runs],
                "write_seconds": round(write_s, 2),
                "note": "page-cache resident files -> pinned staging -> HBM (PCIe); not part of value"}
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def sweep_attention(torch, dev) -> dict:
    """ekernel_paged_attention_bf16 for one sequence: S new rows (1 = decode,
    5 / 4 = MTP verify with 4 / 3 drafts) over L cached positions in 16-token
    blocks, gate from q_proj's output.  Enough distinct caches (>= 512 MB)
    that K and V stream from HBM; GB/s counts K and V once (the kernels'
    bound: 2 * L * n_kv_heads * head_dim * 2 bytes)."""
    from pilm_amd import bindings as abi
    out = {}
    bs, d = 16, 128
    cases = [("qwen3_1p7b", 16, 8, 1, L) for L in (384, 4096, 32768)] + \
            [("qwen3_8b", 32, 8, 1, L) for L in (384, 4096, 32768, 131072)] + \
            [("qwen3_1p7b", 16, 8, 4, 4096), ("qwen3_8b", 32, 8, 5, 4096)]
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    for model, h, hkv, s_rows, L in cases:
        nblk = (L + bs - 1) // bs
        per = 2 * nblk * bs * hkv * d * 2
        copies = max(2, min(64, (512 << 20) // per))
        caches = [(torch.randn(nblk, bs, hkv, d, device=dev, generator=gen).to(torch.bfloat16),
                   torch.randn(nblk, bs, hkv, d, device=dev, generator=gen).to(torch.bfloat16)) for _ in range(copies)]
        ids = torch.randperm(nblk, device=dev, generator=gen).to(torch.int32)
        q = torch.randn(s_rows, h, d, device=dev, generator=gen).to(torch.bfloat16)
        kn = torch.randn(s_rows, hkv, d, device=dev, generator=gen).to(torch.bfloat16)
        vn = torch.randn(s_rows, hkv, d, device=dev, generator=gen).to(torch.bfloat16)
        qg = torch.randn(s_rows, h, 2 * d, device=dev, generator=gen).to(torch.bfloat16)
        o = torch.empty(s_rows, h * d, device=dev, dtype=torch.bfloat16)

        def run():
            abi.set_stream(torch.cuda.current_stream().cuda_stream)
            for kc, vc in caches:
                rc = abi.paged_attention_bf16_ptr(q.data_ptr(), kn.data_ptr(), vn.data_ptr(), kc.data_ptr(),
                                                  vc.data_ptr(), ids.data_ptr(), qg.data_ptr() + 2 * d, o.data_ptr(),
                                                  s_rows, h, hkv, d, L, bs, nblk, nblk, 2 * d)
                if rc != 0:
                    raise RuntimeError(f"ekernel_paged_attention_bf16 failed: rc={rc} ({abi.last_error()})")
        g = capture(torch, run)
        us = time_graph(torch, g, 5, 1) / (5 * copies) * 1e6
        del g, caches
        kv = 2 * L * hkv * d * 2
        out[f"{model}_S{s_rows}_L{L}"] = {"H": h, "Hkv": hkv, "D": d, "S": s_rows, "L": L, "us": round(us, 2),
                                           "kv_GBps": round(kv / us / 1e3, 1)}
    torch.cuda.empty_cache()
    return out


def sweep_fused(torch, dev, reps: int = 20) -> dict:
    """The W4 SwiGLU MLP of one token (Qwen3-1.7B and 8B shapes) fused
    (ekernel_swiglu_w4a16_bf16) vs gate_up GEMV + SwiGLU + down GEMV, and the
    W8A16 lm_head with the argmax epilogue (device outputs) vs the GEMV alone."""
    from pilm_amd import ckernel as ck
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    out = {}

    def timed(fn):
        g = capture(torch, lambda: [fn() for _ in range(reps)])
        sec = time_graph(torch, g, 5, 1)
        del g
        return round(sec / (5 * reps) * 1e6, 2)
    for name, h, i in (("qwen3_1p7b", 2048, 6144), ("qwen3_8b", 4096, 12288)):
        x = torch.randn((1, h), device=dev, generator=gen).to(torch.bfloat16)
        gu, gs = _fmt_weights(torch, dev, "w4row", 2 * i, h, gen)
        dw, ds = _fmt_weights(torch, dev, "w4row", h, i, gen)

        def unfused():
            y = ck.linear_w4a16_bf16(x, gu, gs)
            return ck.linear_w4a16_bf16(ck.swiglu_bf16(y[:, :i], y[:, i:]), dw, ds)
        fused_us = timed(lambda: ck.swiglu_w4a16_bf16(x, gu, gs, dw, ds, i))
        wbytes = 2 * i * (h // 2) + h * (i // 2) + 8 * i + 4 * h
        out[f"swiglu_w4_{name}"] = {"H": h, "I": i, "fused_us": fused_us, "unfused_us": timed(unfused),
                                    "fused_GBps": round(wbytes / fused_us / 1e3, 1)}
        del gu, gs, dw, ds
    for name, k in (("qwen3_1p7b", 2048), ("qwen3_8b", 4096)):
        n = 151936
        x = torch.randn((1, k), device=dev, generator=gen).to(torch.bfloat16)
        w, sc = _fmt_weights(torch, dev, "w8a16", n, k, gen)
        gemv_us = timed(lambda: ck.linear_w8a16_bf16(x, w, sc))
        arg_us = timed(lambda: ck.linear_w8a16_bf16_argmax_device(x, w, sc))
        out[f"lm_head_argmax_w8a16_{name}"] = {"N": n, "K": k, "gemv_us": gemv_us, "gemv_argmax_us": arg_us,
                                               "GBps": round((n * k + 4 * n) / arg_us / 1e3, 1)}
        del w, sc
    torch.cuda.empty_cache()
    return out


def cpu_host() -> dict:
    """CPU model, sockets, physical cores and logical CPUs among the CPUs this
    process may run on (SMT siblings share a core id within a package)."""
    cpus = sorted(os.sched_getaffinity(0))
    cores, packages = set(), set()
    for c in cpus:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            pkg = open(base + "physical_package_id").read().strip()
            core = open(base + "core_id").read().strip()
        except OSError:
            pkg, core = "0", str(c)
        packages.add(pkg)
        cores.add((pkg, core))
    return {"model": _cpu_model(), "sockets": len(packages), "physical_cores": len(cores),
            "logical_cpus": len(cpus)}


def cpu_child(threads: int) -> dict:
    """One thread count (OMP_NUM_THREADS / OMP_PROC_BIND / OMP_PLACES set by
    the parent before this process loaded OpenMP): per shape of one decode
    layer's W4A16-g128 linears plus lm_head (M = 1), 5 warm-up calls and the
    median of >= 20 calls timed with the monotonic clock around the C call."""
    import numpy as np
    from oracle import oracle as O
    from pilm_amd import synth as S
    kind = "reference" if O.ref_available() else "port"
    lib = O.ref_lib() if kind == "reference" else O.oracle_lib()
    fn = lib.ekernel_linear_w4a16g128_bf16 if kind == "reference" else None
    per_shape, tot_bytes, tot_sec = [], 0, 0.0
    for i, (name, n, k) in enumerate(LAYER_SHAPES + [LM_HEAD]):
        x = S.activations_bf16(100 + i, 1, k)
        w = np.random.default_rng(i).integers(0, 256, size=(n, k // 2), dtype=np.uint8)
        sc = S.scales_uniform(200 + i, (n, k // 128))
        out = np.empty((1, n), np.uint16)
        if fn is not None:
            desc = O._Desc(1, n, k)
            args = (ctypes.byref(desc), x.ctypes.data, w.ctypes.data, sc.ctypes.data, out.ctypes.data, 1)
            call = lambda: fn(*args)       # noqa: E731
        else:
            call = lambda: O.linear_w4a16g_bf16(x, w, sc, 128, impl="oracle")   # noqa: E731
        for _ in range(5):
            call()
        times = []
        for _ in range(20):
            t0 = time.clock_gettime(time.CLOCK_MONOTONIC)
            call()
            times.append(time.clock_gettime(time.CLOCK_MONOTONIC) - t0)
        med = float(np.median(times))
        b = alg_bytes(1, n, k)
        per_shape.append({"shape": f"{name} {n}x{k}", "median_ms": round(med * 1e3, 4), "GBps": round(b / med / 1e9, 2)})
        tot_bytes += b
        tot_sec += med
    return {"threads": threads, "kind": kind, "GBps": round(tot_bytes / tot_sec / 1e9, 2), "shapes": per_shape}


def cpu_baseline(budget_s: float = 12.0) -> dict | None:
    """The reference's ekernel_linear_w4a16g128_bf16 (kernels.c compiled from
    its source into oracle/_ref by oracle/Makefile, x86-64-v3 + OpenMP) on this
    host, swept over 1, half and all of the physical cores this process may
    use, each in a child process with OMP_PROC_BIND=close and
    OMP_PLACES=cores.  value: the rate at all physical cores, GB/s of the
    per-shape medians summed over one layer's linears plus lm_head."""
    import subprocess
    host = cpu_host()
    phys = max(1, min(host["physical_cores"], int(os.environ.get("OMP_NUM_THREADS") or host["physical_cores"])))
    sweep = sorted({1, max(1, phys // 2), phys})
    runs = []
    t0 = time.perf_counter()
    for t in sweep:
        env = dict(os.environ, OMP_NUM_THREADS=str(t), OMP_PROC_BIND="close", OMP_PLACES="cores")
        r = subprocess.run([sys.executable, str(Path(__file__).resolve()), "--cpu-child", str(t)], env=env,
                           capture_output=True, text=True, timeout=max(60.0, 10 * budget_s))
        if r.returncode != 0:
            print(r.stderr[-2000:], file=sys.stderr)
            return None
        runs.append(json.loads(r.stdout.strip().splitlines()[-1]))
    top = runs[-1]
    return {"value": top["GBps"], "unit": "GB/s", "cores": top["threads"], "kind": top["kind"],
            "sample": (f"median of 20 calls (after 5 warm-ups) per shape of one Qwen3-1.7B layer's W4A16-g128 "
                       f"linears + lm_head, M=1; threads swept {sweep} in {time.perf_counter() - t0:.1f} s"),
            "cpu": host["model"], "sockets": host["sockets"], "physical_cores": host["physical_cores"],
            "logical_cpus": host["logical_cpus"], "omp": "OMP_PROC_BIND=close OMP_PLACES=cores",
            "build": "kernels.c, gcc -O3 -march=x86-64-v3 -fopenmp (the reference's sources are not on this "
                     "host, so no -march=native build here)",
            "sweep": [{"threads": r["threads"], "GBps": r["GBps"]} for r in runs], "per_shape": top["shapes"]}


def pmc_pass(torch, dev, steps: int) -> None:
    """Eager steps (every dispatch visible to counter collection), then a
    plain copy kernel of known size: out = -x over CALIB_BYTES of fp32."""
    xs, calls = build_step(torch, dev, 1)
    run = launcher(torch, xs, calls, 1)
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    del calls, xs, run
    torch.cuda.empty_cache()
    x = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
    y = torch.empty_like(x)
    for _ in range(3):
        torch.neg(x, out=y)
    torch.cuda.synchronize()
    print(f"[bench] pmc pass: {steps} eager steps of {len(step_shapes())} calls, 3 copy kernels of "
          f"{CALIB_BYTES} B", flush=True)


# Shapes of the per-shape counter pass: (label, format, N, K, M, matrix-core threshold or None)
SHAPE_PMC_CASES = [(f"g128 M=1 {name}", "w4g128", n, k, 1, None) for name, n, k in SHAPES_8B] + [
    ("w8a32 M=1 single 4096x4096", "w8a32", 4096, 4096, 1, None),
    ("w8a32 M=1 q_proj", "w8a32", 8192, 4096, 1, None),
    ("w8a32 M=1 gate_up_proj", "w8a32", 24576, 4096, 1, None),
    ("w8a32 M=1 down_proj", "w8a32", 4096, 12288, 1, None),
    ("w8a16 M=80 gate_up_proj, exact", "w8a16", 24576, 4096, 80, 0),
    ("g128 M=64 gate_up_proj, matrix cores", "w4g128", 24576, 4096, 64, None),
    ("g128 M=1024 gate_up_proj, matrix cores", "w4g128", 24576, 4096, 1024, None),
    ("g128 M=2048 gate_up_proj, matrix cores", "w4g128", 24576, 4096, 2048, None),
    ("w8a32 M=1024 gate_up_proj, matrix cores", "w8a32", 24576, 4096, 1024, None),
]
SHAPE_PMC_COUNTERS = ("SQ_WAVE_CYCLES SQ_WAIT_ANY SQ_BUSY_CYCLES SQ_ACTIVE_INST_VALU SQ_INSTS_VALU SQ_INSTS_MFMA "
                      "SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE")


def shape_pmc_pass(torch, dev, reps: int) -> None:
    """Each shape of SHAPE_PMC_CASES called `reps` times eagerly after a
    marker (a 1-element fill), then the 1 GiB copy kernel: one rocprofv3
    counter pass attributes every dispatch between two markers to a shape."""
    from pilm_amd import bindings as abi
    lib = abi._load_lib()
    marker = torch.empty(1, device=dev)       # (no kernel: the first fill is the first marker)
    gen = torch.Generator(device=dev)
    for label, fmt, n, k, m, thr in SHAPE_PMC_CASES:
        gen.manual_seed(n + k + m)
        w, sc = _fmt_weights(torch, dev, fmt, n, k, gen)
        x = torch.randn((m, k), device=dev, generator=gen)
        x = x if fmt == "w8a32" else x.to(torch.bfloat16)
        out = torch.empty((m, n), dtype=torch.float32 if fmt == "w8a32" else torch.bfloat16, device=dev)
        d = abi.EkernelLinearW8A32Desc(m, n, k)
        fn = getattr(lib, _ENTRY[fmt])
        prev = abi.matrix_core_min_rows()
        if thr is not None:
            abi.set_matrix_core_min_rows(thr)
        try:
            abi.set_stream(torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            marker.fill_(1.0)
            for _ in range(reps):
                rc = fn(ctypes.byref(d), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(w.data_ptr()),
                        ctypes.c_void_p(sc.data_ptr()), ctypes.c_void_p(out.data_ptr()), 6)
                if rc != 0:
                    raise RuntimeError(abi.last_error())
            torch.cuda.synchronize()
        finally:
            abi.set_matrix_core_min_rows(prev)
        print(f"[bench] shape pmc: {label}", flush=True)
        del w, sc, x, out
    marker.fill_(1.0)
    torch.cuda.empty_cache()
    xc = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
    yc = torch.empty_like(xc)
    for _ in range(3):
        torch.neg(xc, out=yc)
    torch.cuda.synchronize()


def shape_counters(sq_csv: str, fetch_csv: str, reps: int) -> str:
    """Markdown table of the shape pass: per call, counter-run time, HBM
    bytes (FETCH_SIZE scaled by the copy kernel) against the algorithmic
    bytes, the share of wave cycles spent waiting, VALU busy, MFMA busy,
    VALU instructions per MFMA, and the shader clock over the call (busy
    cycles per XCD / time)."""
    import csv

    def load(path):
        disp = {}
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                d = disp.setdefault(int(r["Dispatch_Id"]), {"name": r["Kernel_Name"], "t": (int(r["End_Timestamp"]) -
                                                                                            int(r["Start_Timestamp"]))})
                d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        return [disp[i] for i in sorted(disp)]

    def segments(ds):
        segs, cur = [], None
        for d in ds:
            if "FillFunctor" in d["name"]:
                if cur is not None:
                    segs.append(cur)
                cur = []
            elif cur is not None and ("pilm::" in d["name"] or "_ZN4pilm" in d["name"]):
                cur.append(d)
        tail = [d for d in ds if "neg_kernel" in d["name"]]
        return [sg for sg in segs if sg], tail

    sq_segs, _ = segments(load(sq_csv))
    f_segs, f_copy = segments(load(fetch_csv))
    if len(sq_segs) != len(SHAPE_PMC_CASES) or len(f_segs) != len(SHAPE_PMC_CASES) or not f_copy:
        raise SystemExit(f"expected {len(SHAPE_PMC_CASES)} shape segments and the copy kernel")
    ff = CALIB_BYTES / (sum(d["FETCH_SIZE"] for d in f_copy) / len(f_copy) * 1024)
    lines = ["| shape | N x K x M | us per call | HBM GB/s (% of 8 TB/s) | fetch / algorithmic | waiting (% of wave cycles) "
             "| VALU busy % | MFMA busy % | VALU instr per MFMA | clock GHz |", "|---|---|---|---|---|---|---|---|---|---|"]
    for (label, fmt, n, k, m, _), sq, fs in zip(SHAPE_PMC_CASES, sq_segs, f_segs):
        us = sum(d["t"] for d in sq) / reps / 1e3
        fetch = sum(d["FETCH_SIZE"] for d in fs) / reps * 1024 * ff
        alg = _fmt_bytes(fmt, m, n, k)
        tot = {c: sum(d.get(c, 0.0) for d in sq) for c in SHAPE_PMC_COUNTERS.split()}
        # GRBM_GUI_ACTIVE comes summed over the 8 XCDs: per XCD it is the
        # busy cycles the derived VALUBusy / MfmaUtil metrics divide by
        grbm = max(tot["GRBM_GUI_ACTIVE"] / 8, 1.0)
        wait = 100.0 * tot["SQ_WAIT_ANY"] / max(tot["SQ_WAVE_CYCLES"], 1.0)
        valu = 100.0 * tot["SQ_ACTIVE_INST_VALU"] / 256 / grbm
        mfma = 100.0 * tot["SQ_VALU_MFMA_BUSY_CYCLES"] / (grbm * 1024)
        per = (f"{tot['SQ_INSTS_VALU'] / tot['SQ_INSTS_MFMA']:.1f}" if tot["SQ_INSTS_MFMA"] > 0 else "-")
        gbps = alg / (us * 1e-6) / 1e9
        # (for calls of a few us the counter window around the dispatch
        # dominates the busy cycles: no clock for those)
        ghz = f"{grbm / reps / (us * 1e3):.2f}" if us >= 100.0 else "-"
        lines.append(f"| {label} | {n} x {k} x {m} | {us:.2f} | {gbps:.0f} ({gbps / 80:.1f} %) | {fetch / alg:.3f} | "
                     f"{wait:.0f} | {valu:.1f} | {mfma:.1f} | {per} | {ghz} |")
    return "\n".join(lines)


ATTN_PMC_CASE = ("qwen3_8b", 32, 8, 1, 32768)   # model, H, Hkv, S, L (16-token blocks, D = 128)


def attn_pmc_pass(torch, dev, calls: int) -> None:
    """Eager paged-attention calls at one shape (Qwen3-8B heads, one decode
    row over 32768 cached positions), then the plain copy kernel, so that
    FETCH_SIZE / WRITE_SIZE per dispatch of each attention kernel can be set
    against the K and V bytes it has to read."""
    from pilm_amd import bindings as abi
    _, h, hkv, s_rows, L = ATTN_PMC_CASE
    bs, d = 16, 128
    nblk = (L + bs - 1) // bs
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    kc = torch.randn(nblk, bs, hkv, d, device=dev, generator=gen).to(torch.bfloat16)
    vc = torch.randn(nblk, bs, hkv, d, device=dev, generator=gen).to(torch.bfloat16)
    ids = torch.randperm(nblk, device=dev, generator=gen).to(torch.int32)
    q = torch.randn(s_rows, h, d, device=dev, generator=gen).to(torch.bfloat16)
    kn = torch.randn(s_rows, hkv, d, device=dev, generator=gen).to(torch.bfloat16)
    vn = torch.randn(s_rows, hkv, d, device=dev, generator=gen).to(torch.bfloat16)
    qg = torch.randn(s_rows, h, 2 * d, device=dev, generator=gen).to(torch.bfloat16)
    o = torch.empty(s_rows, h * d, device=dev, dtype=torch.bfloat16)
    abi.set_stream(torch.cuda.current_stream().cuda_stream)
    for _ in range(calls):
        rc = abi.paged_attention_bf16_ptr(q.data_ptr(), kn.data_ptr(), vn.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                          ids.data_ptr(), qg.data_ptr() + 2 * d, o.data_ptr(),
                                          s_rows, h, hkv, d, L, bs, nblk, nblk, 2 * d)
        if rc != 0:
            raise RuntimeError(f"ekernel_paged_attention_bf16 failed: rc={rc} ({abi.last_error()})")
    torch.cuda.synchronize()
    del kc, vc
    torch.cuda.empty_cache()
    x = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
    y = torch.empty_like(x)
    for _ in range(3):
        torch.neg(x, out=y)
    torch.cuda.synchronize()
    print(f"[bench] attention pmc pass: {calls} calls S={s_rows} H={h} Hkv={hkv} D={d} L={L}, "
          f"3 copy kernels of {CALIB_BYTES} B", flush=True)


def attn_traffic_summary(fetch_csv: str, write_csv: str) -> dict:
    """Bytes per dispatch of each attention kernel from the two counter runs
    of attn_pmc_pass, scaled by the copy kernel's known size, beside the
    bytes the kernel must move (K for the scores kernel, V for the P.V
    kernel: L * Hkv * D * 2 each)."""
    f = _counter_means(fetch_csv, "FETCH_SIZE")
    w = _counter_means(write_csv, "WRITE_SIZE")
    (cf, _), (cw, _) = _pick(f, "neg_kernel"), _pick(w, "neg_kernel")
    ff, fw = CALIB_BYTES / (cf * 1024), CALIB_BYTES / (cw * 1024)
    _, h, hkv, s_rows, L = ATTN_PMC_CASE
    kv_one = L * hkv * 128 * 2
    out = {"case": {"S": s_rows, "H": h, "Hkv": hkv, "D": 128, "L": L, "block_size": 16},
           "fetch_factor": round(ff, 4), "write_factor": round(fw, 4)}
    for needle in ("attn_scores_kernel", "attn_pv_kernel"):
        hits = [k for k in f if needle in k]
        if not hits:
            continue
        (kf, n) = _pick(f, needle)
        (kw, _) = _pick(w, needle)
        out[needle] = {"fetch_bytes": round(kf * 1024 * ff), "write_bytes": round(kw * 1024 * fw),
                       "must_read_bytes": kv_one, "fetch_over_must": round(kf * 1024 * ff / kv_one, 4),
                       "dispatches": n}
    return out


def _counter_means(csv_path: str, counter: str) -> dict:
    """{kernel name: mean counter value per dispatch} from a rocprofv3
    counter_collection.csv."""
    import csv
    acc = {}
    with open(csv_path, newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            a = acc.setdefault(r["Kernel_Name"], [0.0, 0])
            a[0] += float(r["Counter_Value"])
            a[1] += 1
    return {k: (v[0] / v[1], v[1]) for k, v in acc.items()}


def _pick(means: dict, needle: str):
    hits = [(k, v) for k, v in means.items() if needle in k]
    if len(hits) != 1:
        raise SystemExit(f"expected one kernel matching {needle!r}, found {len(hits)}")
    return hits[0][1]


def _pick_all(means: dict, needles) -> tuple:
    """Dispatch-weighted mean and dispatch count over every kernel whose name
    contains one of `needles`."""
    hits = [v for k, v in means.items() if any(n in k for n in needles)]
    if not hits:
        raise SystemExit(f"no kernel matching {needles!r}")
    total = sum(m * n for m, n in hits)
    count = sum(n for _, n in hits)
    return total / count, count


def traffic_summary(fetch_csv: str, write_csv: str) -> dict:
    """FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of the GEMV and of the
    copy kernel; the copy kernel moves CALIB_BYTES each way, which fixes the
    bytes each counter unit stands for."""
    f = _counter_means(fetch_csv, "FETCH_SIZE")
    w = _counter_means(write_csv, "WRITE_SIZE")
    (gf, nf), (cf, _) = _pick_all(f, GEMV_KERNELS), _pick(f, "neg_kernel")
    (gw, nw), (cw, _) = _pick_all(w, GEMV_KERNELS), _pick(w, "neg_kernel")
    ff, fw = CALIB_BYTES / (cf * 1024), CALIB_BYTES / (cw * 1024)
    fetch_b, write_b = gf * 1024 * ff, gw * 1024 * fw
    step_alg = sum(alg_bytes(1, n, k) for (_, n, k) in step_shapes())
    return {"traffic": round(fetch_b + write_b), "fetch_bytes": round(fetch_b), "write_bytes": round(write_b),
            "alg_bytes_per_launch": round(step_alg / len(step_shapes())),
            "fetch_kib_raw": round(gf, 3), "write_kib_raw": round(gw, 3),
            "copy_fetch_kib_raw": round(cf, 3), "copy_write_kib_raw": round(cw, 3),
            "fetch_factor": round(ff, 4), "write_factor": round(fw, 4),
            "dispatches": [nf, nw], "source_sha256": source_hash()}


def stats_summary(stats_csv: str, top: int = 8) -> str:
    import csv
    rows = list(csv.DictReader(open(stats_csv, newline="")))
    lines = ["| kernel | calls | total ms | avg us | min us | max us | % |", "|---|---|---|---|---|---|---|"]
    for r in rows[:top]:
        name = r["Name"]
        short = name.replace("(anonymous namespace)::", "").split("(")[0].replace("void ", "")
        if len(short) > 90:
            short = short[:87] + "..."
        lines.append(f"| `{short}` | {r['Calls']} | {float(r['TotalDurationNs']) / 1e6:.3f} | "
                     f"{float(r['AverageNs']) / 1e3:.3f} | {float(r['MinNs']) / 1e3:.3f} | "
                     f"{float(r['MaxNs']) / 1e3:.3f} | {float(r['Percentage']):.2f} |")
    return "\n".join(lines)


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
    ap.add_argument("--sweep", nargs="?", const="g128", default=None,
                    help="add per-shape sweeps: comma list of g128,w4row,w8a32,w8a16,gemm,fused,attention,load or 'all'")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--pmc-pass", action="store_true")
    ap.add_argument("--traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"))
    ap.add_argument("--stats-summary", metavar="STATS_CSV")
    ap.add_argument("--attn-pmc-pass", action="store_true")
    ap.add_argument("--shape-pmc-pass", action="store_true",
                    help="the Qwen3-8B GEMV / GEMM / verify shapes, one counter pass")
    ap.add_argument("--shape-counters", nargs=2, metavar=("SQ_CSV", "FETCH_CSV"),
                    help="counter CSVs of two --shape-pmc-pass runs -> markdown table")
    ap.add_argument("--attn-traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"))
    ap.add_argument("--layout", choices=("fused", "separate"), default="fused",
                    help="q/k/v and gate/up as one matrix each (the decoder's layout) or one call per projection")
    ap.add_argument("--no-decode", action="store_true", help="skip the whole-decoder tok/s measurement")
    ap.add_argument("--cpu-child", type=int, metavar="THREADS", help=argparse.SUPPRESS)
    args = ap.parse_args(argv)
    global LAYER_SHAPES
    LAYER_SHAPES = LAYER_SHAPES_FUSED if args.layout == "fused" else LAYER_SHAPES_SEPARATE
    if args.cpu_child:
        print(json.dumps(cpu_child(args.cpu_child)))
        return 0
    if args.traffic:
        rec = traffic_summary(*args.traffic)
        TRAFFIC_FILE.parent.mkdir(exist_ok=True)
        TRAFFIC_FILE.write_text(
            f"# HBM traffic per launch of {GEMV_KERNEL}, Qwen3-1.7B W4A16-g128 decode step (M=1)\n"
            "# passes: rocprofv3 --pmc FETCH_SIZE (then WRITE_SIZE) --output-format csv -d DIR -o run "
            "-- python bench.py --pmc-pass --steps 2\n"
            f"# then:  python bench.py --traffic DIR_F/run_counter_collection.csv DIR_W/run_counter_collection.csv\n"
            f"# counter KiB x (copy kernel's known {CALIB_BYTES} B / its counter KiB) = bytes\n"
            + json.dumps(rec) + "\n")
        print(json.dumps(rec))
        return 0
    if args.stats_summary:
        print(stats_summary(args.stats_summary))
        return 0
    if args.attn_traffic:
        print(json.dumps(attn_traffic_summary(*args.attn_traffic)))
        return 0
    if args.shape_counters:
        print(shape_counters(*args.shape_counters, reps=args.steps))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU: there is no multi-GPU path (asked for --gpus {args.gpus}); "
              "the decode GEMV would shard by output rows, each GPU holding W[N/G, K] and its scales",
              file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    if args.pmc_pass:
        pmc_pass(torch, dev, args.steps)
        return 0
    if args.attn_pmc_pass:
        attn_pmc_pass(torch, dev, args.steps)
        return 0
    if args.shape_pmc_pass:
        shape_pmc_pass(torch, dev, args.steps)
        return 0
    m = 1
    print(f"[bench] building step: {len(step_shapes())} W4A16-g128 linears, M={m}", flush=True)
    xs, calls = build_step(torch, dev, m)
    run = launcher(torch, xs, calls, m)
    step_bytes = sum(alg_bytes(m, n, k) for (_, n, k, *_rest) in calls)
    g = capture(torch, run)
    print(f"[bench] graph captured; timing {args.steps} steps after {args.warmup} warmup", flush=True)
    sec, gpu_sec = time_graph(torch, g, args.steps, args.warmup, events=True)
    ms_per_step = sec / args.steps * 1e3
    value = step_bytes * args.steps / sec / 1e9
    roof = roofline(gpu_sec, args.steps * len(calls), step_bytes / len(calls))

    # eager (no graph) step time, for reference
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        run()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) / 3 * 1e3

    del g
    copy_gbs = copy_peak(torch, dev)
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
        "config": {"workload": "Qwen3-1.7B W4A16-g128 decode linears, one token (28 layers x "
                               f"{len(LAYER_SHAPES)} + lm_head, {args.layout} q/k/v and gate/up)",
                   "M": m, "calls_per_step": len(calls), "alg_bytes_per_step": step_bytes,
                   "entry_point": "ekernel_linear_w4a16g128_bf16", "launch": "HIP graph replay"},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "hbm_copy_GBps": round(copy_gbs, 1),
        "pct_of_copy_peak": round(100 * value / copy_gbs, 2),
        "decode_linear_tok_s": round(1e3 / ms_per_step, 1),
        "eager_ms_per_step": round(eager_ms, 3),
        "roofline": roof,
    }
    if not args.no_decode:
        del calls, xs, run
        torch.cuda.empty_cache()
        print("[bench] whole decoder: Qwen3-1.7B W4A16-g128, 128-token prompt, 256 greedy tokens", flush=True)
        dec = decode_bench(torch, dev)
        out["decode_tok_s"] = dec["decode_tok_s"]
        out["decode"] = dec
        calls = xs = run = None
    if args.sweep:
        sections = ("g128", "w4row", "w8a32", "w8a16", "gemm", "gemm_fp16", "fused", "attention", "load", "verify",
                    "verify_step", "verify_step_8b") \
            if args.sweep == "all" \
            else tuple(args.sweep.split(","))
        print(f"[bench] sweeps: {', '.join(sections)}", flush=True)
        del calls, xs, run
        torch.cuda.empty_cache()
        out["sweep"] = sweep(torch, dev, sections)
    if not args.no_cpu:
        print("[bench] cpu baseline", flush=True)
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
