"""Write the greedy-decode fixtures by running piLM's own engine on the CPU.

Development container only: this script imports the reference from
/root/reference/src (its Qwen3Model, QuantizedW4A16Linear, quantizer,
PhysicalKVCache, Scheduler and Engine.generate) together with the
reference's C library built from its own sources by `make -C oracle
ref_full`.  The GPU tests read only the JSON files it writes.

What is run, per configuration:
  * weights: every tensor ~N(0, 0.02) from pilm_amd.synth_model (seeded,
    bit-identical on CPU and GPU); every Linear (q/k/v/o, gate/up/down and
    lm_head) quantized by the reference's quantize_weight_i4_grouped_chunked
    (src/runtime/ckernel.py:124-161) with group 128 and wrapped in its
    QuantizedW4A16Linear (src/models/base/linear.py:267-340); norms and the
    embedding bf16;
  * the model: the reference's Qwen3Model (src/models/qwen3/model.py:76-127)
    with every layer full attention (gated q_proj, q/k GemmaRMSNorm, rope with
    partial_rotary_factor 1.0, theta 1e6), bf16;
  * the run: Engine.generate (src/engine.py:319-664) with temperature 0 and
    top_k 0, a uniform random prompt, 16-token KV blocks and its scheduler
    (prefill in 16-token chunks, src/engine.py:218), driven through an Engine
    object assembled here without its file loaders and with a tokenizer stub
    whose decode returns the token id.  The engine's loop counts each prefill
    chunk as a step (src/engine.py:383), so it is asked for
    new_tokens + chunks - 1 tokens and the first new_tokens are kept.

torch runs with its AVX2 kernels (ATEN_CPU_CAPABILITY=avx2) and oneDNN off:
the reference was measured on an i9-14900K (docs/runtime_status.md:361-365),
which has neither AVX-512 nor bf16 matrix instructions, so torch used its own
AVX2 kernels there.  These settings fix the summation orders the device
decoder reproduces (softmax's 8-lane reduction and the bf16 batched matrix
products of the attention).

Recorded: prompt and generated token ids; for every lm_head call the SHA-256
of its bf16 logits, its argmax and the top-two values; the SHA-256 of every
quantized tensor (qweight, scales); the SHA-256 of the rope cos/sin tables
for every position used.

    python tests/golden/gen_decode_fixture.py [tiny|qwen3_1p7b|all]
"""
from __future__ import annotations

import os
import sys

os.environ["ATEN_CPU_CAPABILITY"] = "avx2"          # before torch is imported
os.environ.setdefault("OMP_NUM_THREADS", "8")

import hashlib
import json
import time
from pathlib import Path
from types import SimpleNamespace

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
REF_SRC = Path("/root/reference/src")
REF_LIB = REPO / "oracle" / "_ref" / "libecpu_ref_full.so"

CONFIGS = {
    "tiny": dict(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=128, intermediate=512, vocab=4096,
                 prompt=40, new_tokens=48, seed=11),
    "qwen3_1p7b": dict(layers=28, hidden=2048, heads=16, kv_heads=8, head_dim=128, intermediate=6144,
                       vocab=151936, prompt=128, new_tokens=256, seed=1),
}
COMMON = dict(eps=1e-6, rope_theta=1e6, partial_rotary=1.0, block_size=16, group_size=128, std=0.02)


def _say(msg):
    print(msg, flush=True)


def _sha(t) -> str:
    return hashlib.sha256(t.contiguous().view(-1).view(__import__("torch").uint8).numpy().tobytes()).hexdigest()


def build_and_run(name: str) -> dict:
    import torch
    import torch.nn as nn
    torch.backends.mkldnn.enabled = False
    assert torch.backends.cpu.get_cpu_capability() == "AVX2", torch.backends.cpu.get_cpu_capability()
    if not REF_LIB.exists():
        raise SystemExit(f"{REF_LIB} missing: run make -C oracle ref_full")
    os.environ["PILM_ECPU_LIB"] = str(REF_LIB)
    sys.path.insert(0, str(REF_SRC))
    sys.path.insert(0, str(REPO))
    from pilm_amd import synth_model as SM
    from engine import Engine
    from models.qwen3.model import Qwen3Model
    from models.base.linear import QuantizedW4A16Linear
    from models.base.layers import _rope_inv_freq, _rope_cos_sin
    from runtime.ckernel import quantize_weight_i4_grouped_chunked
    from runtime.scheduler import Scheduler, KVCacheManager
    from runtime.kvcache import PhysicalKVCache

    c = dict(CONFIGS[name], **COMMON)
    L, H, V = c["layers"], c["hidden"], c["vocab"]
    rope = SimpleNamespace(rope_theta=c["rope_theta"], partial_rotary_factor=c["partial_rotary"],
                           mrope_section=None, mrope_interleaved=True)
    tc = SimpleNamespace(hidden_size=H, rms_norm_eps=c["eps"], num_attention_heads=c["heads"],
                         num_key_value_heads=c["kv_heads"], head_dim=c["head_dim"], rope=rope,
                         intermediate_size=c["intermediate"], vocab_size=V, num_hidden_layers=L,
                         layer_types=["full_attention"] * L, dtype="bfloat16")
    config = SimpleNamespace(text_config=tc, num_layers=L)
    with torch.device("meta"):
        model = Qwen3Model(config)
    ids = SM.tensor_ids(L)
    seed = c["seed"]
    qhash = {}

    def bf16_param(tname, shape):
        return nn.Parameter(SM.normal_f32(seed, ids[tname], shape, c["std"]).to(torch.bfloat16),
                            requires_grad=False)

    def quantized(tname, lin):
        out_f, in_f = lin.weight.shape
        w = SM.normal_f32(seed, ids[tname], (out_f, in_f), c["std"])
        q, s = quantize_weight_i4_grouped_chunked(w, group_size=c["group_size"])
        qhash[tname] = [_sha(q), _sha(s)]
        return QuantizedW4A16Linear(q, s, in_f)

    t0 = time.time()
    model.embed_tokens.weight = bf16_param("embed_tokens", (V, H))
    for i, layer in enumerate(model.layers):
        p = f"layers.{i}."
        layer.input_layernorm.weight = bf16_param(p + "input_layernorm", (H,))
        layer.post_attention_layernorm.weight = bf16_param(p + "post_attention_layernorm", (H,))
        attn = layer.self_attn
        attn.q_norm.weight = bf16_param(p + "self_attn.q_norm", (c["head_dim"],))
        attn.k_norm.weight = bf16_param(p + "self_attn.k_norm", (c["head_dim"],))
        for proj in ("q_proj", "k_proj", "v_proj", "o_proj"):
            setattr(attn, proj, quantized(p + "self_attn." + proj, getattr(attn, proj)))
        for proj in ("gate", "up", "down"):
            setattr(layer.mlp, proj, quantized(p + "mlp." + proj, getattr(layer.mlp, proj)))
        _say(f"[fixture {name}] layer {i} materialised ({time.time() - t0:.1f} s)")
    model.norm.weight = bf16_param("norm", (H,))
    model.lm_head = quantized("lm_head", model.lm_head)
    model.eval()

    # Engine without its file loaders (src/engine.py:105-265 builds the same parts)
    class _Tok:
        eos_id = -1

        def decode(self, token_list):
            return str(int(token_list[0]))

    block = c["block_size"]
    n_ctx = c["prompt"] + c["new_tokens"] + 2 * block
    num_blocks = max(64, (n_ctx + block - 1) // block)
    eng = object.__new__(Engine)
    eng.model, eng.config, eng.dtype = model, config, torch.bfloat16
    eng.quantize, eng.quantization_policy, eng.mtp_draft = "w4a16g128-static", "all", None
    eng.ckernel_available, eng.ckernel_info = True, {}
    eng.tokenizer = _Tok()
    eng.block_size = block
    eng.kv_manager = KVCacheManager(num_blocks, block, enable_caching=False)
    eng.scheduler = Scheduler(eng.kv_manager, max_num_batched_tokens=block)
    eng.physical_kv = PhysicalKVCache(num_layers=L, num_blocks=num_blocks, block_size=block,
                                      num_kv_heads=c["kv_heads"], head_dim=c["head_dim"], dtype=torch.bfloat16)
    eng._req_counter, eng.last_stats = 0, {}

    calls = []

    def hook(_mod, _inp, out):
        row = out.reshape(-1, out.shape[-1])[-1]
        f = row.to(torch.float32)
        top = torch.topk(f, 2)
        calls.append({"sha": _sha(row), "argmax": int(torch.argmax(f).item()),
                      "top": [float(top.values[0]), float(top.values[1])]})
    model.lm_head.register_forward_hook(hook)

    prompt = SM.token_ids(seed, c["prompt"], V).tolist()
    chunks = (c["prompt"] + block - 1) // block
    ask = c["new_tokens"] + chunks - 1
    _say(f"[fixture {name}] generating {c['new_tokens']} tokens after a {c['prompt']}-token prompt")
    t1 = time.time()
    with torch.no_grad():
        out = [int(s) for s in eng.generate(prompt, max_new_tokens=ask, temperature=0.0, top_k=0)]
    _say(f"[fixture {name}] generated {len(out)} tokens in {time.time() - t1:.1f} s")
    tokens = out[:c["new_tokens"]]
    # lm_head calls: one per prefill chunk (the last one yields token 0), then one per decode step
    used = calls[chunks - 1:chunks - 1 + c["new_tokens"]]
    assert [u["argmax"] for u in used] == tokens, "hooked logits disagree with the engine's tokens"

    positions = c["prompt"] + c["new_tokens"]
    inv = _rope_inv_freq(torch.device("cpu"), int(c["head_dim"] * c["partial_rotary"]) // 2, c["rope_theta"])
    cos, sin = _rope_cos_sin(torch.arange(positions, dtype=torch.long), inv, c["rope_theta"])
    return {
        "config": c, "name": name,
        "generated_with": {"torch": torch.__version__, "cpu_capability": torch.backends.cpu.get_cpu_capability(),
                           "mkldnn": torch.backends.mkldnn.enabled, "engine_max_new_tokens": ask,
                           "prefill_chunks": chunks},
        "prompt": prompt, "tokens": tokens,
        "logits": used, "prefill_logits": calls[:chunks - 1],
        "rope": {"positions": positions, "cos_sha": _sha(cos), "sin_sha": _sha(sin)},
        "quantized_sha": qhash,
    }


def main():
    which = sys.argv[1] if len(sys.argv) > 1 else "all"
    names = list(CONFIGS) if which == "all" else [which]
    for name in names:
        res = build_and_run(name)
        path = HERE / f"decode_{name}.json"
        path.write_text(json.dumps(res, indent=1))
        _say(f"[fixture {name}] wrote {path.name}: tokens[:12] = {res['tokens'][:12]}")


if __name__ == "__main__":
    main()
