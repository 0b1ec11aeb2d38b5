"""Quantized-weight cache files and bundles, uploaded once to HBM.

Mirrors the quantized-linear cache of piLM's src/models/qwen3/weights.py
(`_quant_cache_path` :59-62, `_maybe_load_quantized_linear_cache` :200-249,
`_save_quantized_linear_cache` :252-266) and the bundle layout written by
scripts/export_pilm_quant_bundle_v2.py:97-186 (`pilm_quant_manifest.json`,
one cache file per quantized Linear under `linear_w4a16/` or
`linear_w8a32/`).  The file formats are unchanged; what changes is where the
tensors go: their bytes are read straight from the safetensors files into
HBM (`eram_hip_load_file`: pinned staging, copy stream, read/copy overlap),
without materialising CPU tensors, and a whole bundle lands in one HBM arena
that every kernel then reads in place.
"""
from __future__ import annotations

import hashlib
import json
import os
import struct
import time
from pathlib import Path

import torch

from . import bindings as abi

W4_FORMATS = {"w4a16", "w4a16g32", "w4a16g128"}
_DTYPES = {"U8": torch.uint8, "I8": torch.int8, "F32": torch.float32, "I32": torch.int32, "BF16": torch.bfloat16,
           "F16": torch.float16}
_ALIGN = 256


def quant_cache_path(cache_dir, src_name: str) -> Path:
    """weights.py:59-62: `{sha1(src)[:16]}-{src with / and . -> _}.safetensors`."""
    digest = hashlib.sha1(src_name.encode("utf-8")).hexdigest()[:16]
    leaf = src_name.replace("/", "_").replace(".", "_")
    return Path(cache_dir) / f"{digest}-{leaf}.safetensors"


def save_quantized_linear_cache(cache_file, qweight: torch.Tensor, scales: torch.Tensor,
                                in_features: int | None = None) -> None:
    """weights.py:252-266: payload qweight / scales (+ in_features int32[1]
    for W4), written to a temporary name and renamed."""
    from safetensors.torch import save_file

    cache_file = Path(cache_file)
    cache_file.parent.mkdir(parents=True, exist_ok=True)
    tmp_file = cache_file.with_suffix(cache_file.suffix + ".tmp")
    payload = {"qweight": qweight.detach().cpu().contiguous(), "scales": scales.detach().cpu().contiguous()}
    if in_features is not None:
        payload["in_features"] = torch.tensor([int(in_features)], dtype=torch.int32)
    save_file(payload, str(tmp_file))
    os.replace(tmp_file, cache_file)


def read_safetensors_header(path) -> dict:
    """{name: (torch dtype, shape, absolute file offset, nbytes)} of a
    safetensors file (8-byte little-endian header length, JSON header, data)."""
    with open(path, "rb") as f:
        (n,) = struct.unpack("<Q", f.read(8))
        header = json.loads(f.read(n))
    base = 8 + n
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        begin, end = meta["data_offsets"]
        out[name] = (_DTYPES[meta["dtype"]], tuple(meta["shape"]), base + begin, end - begin)
    return out


def _expected(quant_format: str, out_features: int, in_features: int):
    """weights.py:216-232: the payload shapes and dtypes a cache must have."""
    if quant_format in W4_FORMATS:
        wshape = (out_features, (in_features + 1) // 2)
        sshape = ((out_features, (in_features + 31) // 32) if quant_format == "w4a16g32"
                  else (out_features, (in_features + 127) // 128) if quant_format == "w4a16g128"
                  else (out_features,))
        return wshape, torch.uint8, sshape
    return (out_features, in_features), torch.int8, (out_features,)


def check_quantized_linear_cache(header: dict, quant_format: str, out_features: int, in_features: int) -> bool:
    """weights.py:213-240: the checks that make a cache file usable."""
    if "qweight" not in header or "scales" not in header:
        return False
    wshape, wdtype, sshape = _expected(quant_format, out_features, in_features)
    qd, qs = header["qweight"][:2]
    sd, ss = header["scales"][:2]
    if qs != wshape or ss != sshape or qd != wdtype or sd != torch.float32:
        return False
    return True


def _cached_in_features(path, header) -> int | None:
    if "in_features" not in header:
        return None
    dtype, shape, off, nbytes = header["in_features"]
    with open(path, "rb") as f:
        f.seek(off)
        raw = f.read(nbytes)
    return int(torch.frombuffer(bytearray(raw), dtype=dtype).reshape(-1)[0].item())


def load_quantized_linear_cache(cache_file, out_features: int, in_features: int, quant_format: str = "w8a32",
                                device="cuda"):
    """weights.py:200-249 on the device: (qweight, scales) tensors in HBM, or
    None when the file is missing or fails the reference's checks."""
    cache_file = Path(cache_file)
    if not cache_file.exists():
        return None
    header = read_safetensors_header(cache_file)
    if not check_quantized_linear_cache(header, quant_format, out_features, in_features):
        return None
    if quant_format in W4_FORMATS:
        cached = _cached_in_features(cache_file, header)
        if cached is not None and cached != in_features:
            return None
    tensors = {}
    ranges = []
    for name in ("qweight", "scales"):
        dtype, shape, off, nbytes = header[name]
        t = torch.empty(shape, dtype=dtype, device=device)
        tensors[name] = t
        ranges.append((off, nbytes, t.data_ptr()))
    # the upload runs on the library's own copy stream: order it after the
    # work torch's stream has queued on memory these fresh tensors may reuse
    torch.cuda.current_stream(device).synchronize()
    rc = abi.eram_load_file(str(cache_file), ranges)
    if rc != 0:
        raise RuntimeError(f"eram_hip_load_file failed: rc={rc} ({abi.last_error()})")
    return tensors["qweight"], tensors["scales"]


class QuantBundle:
    """The quantized Linears of a piLM bundle, resident in one HBM arena.

    `linears` maps each quantized source tensor name (manifest
    `quantized_linear_sources`) to (qweight, scales, in_features): views of
    the arena, each tensor 256-byte aligned.  `stats` records the bytes, the
    files and the upload time."""

    def __init__(self, bundle_dir, device="cuda"):
        bundle_dir = Path(bundle_dir)
        manifest = json.loads((bundle_dir / "pilm_quant_manifest.json").read_text(encoding="utf-8"))
        self.manifest = manifest
        self.quant_format = manifest["quant_format"]
        linear_dir = bundle_dir / manifest["linear_subdir"]
        plan = []   # (src, file, header)
        total = 0
        for src in manifest["quantized_linear_sources"]:
            path = linear_dir / quant_cache_path(linear_dir, src).name
            header = read_safetensors_header(path)
            if "qweight" not in header or "scales" not in header:
                raise ValueError(f"{path}: not a quantized-linear cache file")
            for name in ("qweight", "scales"):
                total += -(-header[name][3] // _ALIGN) * _ALIGN
            plan.append((src, path, header))
        self.arena = torch.empty((max(total, 1),), dtype=torch.uint8, device=device)
        # uploads run on the library's copy stream: order them after torch's
        # queued work on memory the fresh arena may reuse
        torch.cuda.current_stream(self.arena.device).synchronize()
        self.linears = {}
        off = 0
        t0 = time.perf_counter()
        for src, path, header in plan:
            views, ranges = {}, []
            for name in ("qweight", "scales"):
                dtype, shape, foff, nbytes = header[name]
                view = self.arena[off:off + nbytes].view(dtype).view(shape)
                views[name] = view
                ranges.append((foff, nbytes, view.data_ptr()))
                off += -(-nbytes // _ALIGN) * _ALIGN
            rc = abi.eram_load_file(str(path), ranges)
            if rc != 0:
                raise RuntimeError(f"eram_hip_load_file({path}) failed: rc={rc} ({abi.last_error()})")
            in_features = _cached_in_features(path, header)
            if in_features is None:   # W8: K is the row length
                in_features = views["qweight"].shape[1]
            self.linears[src] = (views["qweight"], views["scales"], in_features)
        seconds = time.perf_counter() - t0
        self.stats = {"linears": len(plan), "bytes": off, "seconds": seconds,
                      "GBps": off / seconds / 1e9 if seconds > 0 else 0.0}

    def module(self, src: str):
        """The quantized Linear module of one source tensor, its buffers the
        arena views (no copy)."""
        from .linear import QuantizedW4A16Linear, QuantizedW8A32Linear
        qweight, scales, in_features = self.linears[src]
        if self.quant_format in W4_FORMATS:
            return QuantizedW4A16Linear(qweight, scales, in_features)
        return QuantizedW8A32Linear(qweight, scales)


def write_bundle(bundle_dir, quant_format: str, linears: dict) -> Path:
    """A bundle in the export_pilm_quant_bundle_v2.py layout holding only the
    quantized Linears: {src_name: (qweight, scales, in_features or None)}
    written as cache files under linear_w4a16/ or linear_w8a32/, plus the
    manifest fields the loaders read.  (Residual / MTP tensors and tokenizer
    files are the engine's, not this path's.)"""
    bundle_dir = Path(bundle_dir)
    subdir = "linear_w4a16" if quant_format in W4_FORMATS else "linear_w8a32"
    for src, (qweight, scales, in_features) in linears.items():
        save_quantized_linear_cache(quant_cache_path(bundle_dir / subdir, src), qweight, scales, in_features)
    manifest = {"format": "pilm-quant-bundle-v1", "quantize": f"{quant_format}-all", "quant_format": quant_format,
                "linear_subdir": subdir, "quantized_linear_tensors": len(linears),
                "quantized_linear_sources": sorted(linears), "residual_exports": [], "mtp_exports": []}
    (bundle_dir / "pilm_quant_manifest.json").write_text(json.dumps(manifest, indent=2), encoding="utf-8")
    return bundle_dir
