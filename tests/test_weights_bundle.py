"""Quantized-weight cache files and bundles (pilm_amd.weights): the file
formats on the CPU, the upload to HBM and the modules built on it on the GPU."""
from __future__ import annotations

import hashlib
import json
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402
from pilm_amd import synth as S  # noqa: E402
from pilm_amd import weights as Wt  # noqa: E402


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def test_cache_path_naming(tmp_path):
    name = "model.layers.0.mlp.down_proj.weight"
    p = Wt.quant_cache_path(tmp_path, name)
    assert p.parent == tmp_path
    assert p.name == hashlib.sha1(name.encode()).hexdigest()[:16] + "-model_layers_0_mlp_down_proj_weight.safetensors"
    assert Wt.quant_cache_path(tmp_path, "a/b.c").name.endswith("-a_b_c.safetensors")


def test_header_matches_safetensors_library(tmp_path):
    from safetensors import safe_open
    q = torch.from_numpy(S.weights_i4_packed(1, 33, 70))
    s = torch.from_numpy(S.scales_uniform(2, (33,), fp16_round=False))
    f = tmp_path / "x.safetensors"
    Wt.save_quantized_linear_cache(f, q, s, 70)
    hdr = Wt.read_safetensors_header(f)
    raw = f.read_bytes()
    with safe_open(str(f), framework="pt", device="cpu") as sf:
        assert set(sf.keys()) == set(hdr)
        for name in sf.keys():
            t = sf.get_tensor(name)
            dtype, shape, off, nbytes = hdr[name]
            assert (t.dtype, tuple(t.shape)) == (dtype, shape)
            assert raw[off:off + nbytes] == t.contiguous().view(torch.uint8).numpy().tobytes()
    assert Wt._cached_in_features(f, hdr) == 70


def test_cache_checks_follow_the_reference(tmp_path):
    f = tmp_path / "w4.safetensors"
    Wt.save_quantized_linear_cache(f, torch.zeros((8, 35), dtype=torch.uint8), torch.ones(8), 70)
    h = Wt.read_safetensors_header(f)
    assert Wt.check_quantized_linear_cache(h, "w4a16", 8, 70)
    assert Wt.check_quantized_linear_cache(h, "w4a16", 8, 69)          # ceil(69/2) = 35 too
    assert not Wt.check_quantized_linear_cache(h, "w4a16", 8, 72)      # packed width 36
    assert not Wt.check_quantized_linear_cache(h, "w4a16g128", 8, 70)  # scales must be [8, 1]
    assert not Wt.check_quantized_linear_cache(h, "w8a32", 8, 35)      # int8 expected
    g = tmp_path / "g.safetensors"
    Wt.save_quantized_linear_cache(g, torch.zeros((8, 35), dtype=torch.uint8), torch.ones(8, 3), 70)
    assert Wt.check_quantized_linear_cache(Wt.read_safetensors_header(g), "w4a16g32", 8, 70)
    w8 = tmp_path / "w8.safetensors"
    Wt.save_quantized_linear_cache(w8, torch.zeros((8, 70), dtype=torch.int8), torch.ones(8))
    assert Wt.check_quantized_linear_cache(Wt.read_safetensors_header(w8), "w8a32", 8, 70)


def test_bundle_manifest_layout(tmp_path):
    lin = {"layers.0.q.weight": (torch.zeros((4, 8), dtype=torch.uint8), torch.ones(4), 16)}
    Wt.write_bundle(tmp_path, "w4a16", lin)
    m = json.loads((tmp_path / "pilm_quant_manifest.json").read_text())
    assert m["linear_subdir"] == "linear_w4a16" and m["quant_format"] == "w4a16"
    assert m["quantized_linear_sources"] == ["layers.0.q.weight"]
    assert Wt.quant_cache_path(tmp_path / "linear_w4a16", "layers.0.q.weight").exists()


# ------------------------------------------------------------------ GPU

@pytest.mark.gpu
def test_cache_upload_is_byte_exact(tmp_path, dev):
    q = torch.from_numpy(S.weights_i4_packed(3, 1000, 3000))
    s = torch.from_numpy(S.scales_uniform(4, (1000, 24), fp16_round=False))
    f = tmp_path / "g128.safetensors"
    Wt.save_quantized_linear_cache(f, q, s, 3000)
    _say("[gpu] cache upload")
    got = Wt.load_quantized_linear_cache(f, 1000, 3000, "w4a16g128", dev)
    assert got is not None and got[0].device.type == "cuda"
    assert torch.equal(got[0].cpu(), q) and torch.equal(got[1].cpu(), s)
    assert Wt.load_quantized_linear_cache(f, 1000, 2990, "w4a16g128", dev) is None   # in_features differs
    assert Wt.load_quantized_linear_cache(tmp_path / "missing.safetensors", 1, 1, "w8a32", dev) is None


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["w4a16", "w8a32"])
def test_bundle_resident_and_modules_exact(fmt, tmp_path, dev):
    shapes = {"model.layers.0.self_attn.q_proj.weight": (300, 512), "model.layers.0.mlp.down_proj.weight": (64, 768),
              "model.layers.1.self_attn.o_proj.weight": (17, 256)}
    lin = {}
    for i, (name, (n, k)) in enumerate(shapes.items()):
        if fmt == "w4a16":
            lin[name] = (torch.from_numpy(S.weights_i4_packed(10 + i, n, k)),
                         torch.from_numpy(S.scales_uniform(20 + i, (n,), fp16_round=False)), k)
        else:
            lin[name] = (torch.from_numpy(S.weights_i8(10 + i, n, k)),
                         torch.from_numpy(S.scales_uniform(20 + i, (n,), fp16_round=False)), None)
    Wt.write_bundle(tmp_path, fmt, lin)
    _say(f"[gpu] bundle {fmt}")
    b = Wt.QuantBundle(tmp_path, dev)
    assert b.stats["linears"] == 3 and set(b.linears) == set(shapes)
    for name, (q, s, k) in lin.items():
        qd, sd, kd = b.linears[name]
        assert qd.data_ptr() % 256 == 0 and sd.data_ptr() % 256 == 0
        assert torch.equal(qd.cpu(), q) and torch.equal(sd.cpu(), s) and kd == shapes[name][1]
        mod = b.module(name)
        x = S.activations_bf16(30, 2, shapes[name][1])
        xd = torch.from_numpy(x.view(np.int16)).to(dev).view(torch.bfloat16)
        y = mod(xd).view(torch.int16).cpu().numpy().view(np.uint16)
        ref = (O.linear_w4a16_bf16(x, q.numpy(), s.numpy()) if fmt == "w4a16"
               else O.linear_w8a16_bf16(x, q.numpy(), s.numpy()))
        assert np.array_equal(y, ref), name
