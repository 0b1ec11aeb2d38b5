"""Qwen3 decoder on one MI355X: piLM's Qwen3Model and its greedy decode loop
with every step on the device.

Mirrors src/models/qwen3/model.py:10-127 (TransformerBlock, Qwen3Model),
src/models/qwen3/attention.py:46-141 (FullAttention: gated q_proj, q/k
GemmaRMSNorm, rope, paged KV, sigmoid gate) and the greedy path of
src/engine.py:319-664 (prefill in block-aligned chunks of at most one
16-token block, one token per step after it, argmax of the bf16 logits):
  * linears: the quantized-linear entry points of the HIP libecpu (W4A16 g128
    here), bit-identical to the reference's C kernels; q/k/v and gate/up are
    row-concatenated into one matrix each, which leaves every output row's
    arithmetic unchanged;
  * everything else: the decoder-step entry points (ekernel_rmsnorm_gemma_bf16,
    ekernel_qk_norm_rope_bf16, ekernel_attention_exact_bf16,
    ekernel_silu_mul_bf16, ekernel_greedy_step_bf16), which reproduce the
    reference's torch CPU roundings;
  * the rope tables are computed once on the host with torch's CPU operations
    in the reference's order (layers.py:50-78) and uploaded.
A decode step is captured once into a HIP graph; its kernels read the
position from a device state word that the greedy step advances, so
successive replays generate successive tokens with no host work in between.

There is no CPU path: the library must be built and a GPU present.
"""
from __future__ import annotations

import ctypes
import hashlib
from dataclasses import dataclass, field

import torch

from . import bindings as abi
from . import ckernel
from . import synth_model as SM


@dataclass
class Qwen3Config:
    layers: int = 28
    hidden: int = 2048
    heads: int = 16
    kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 6144
    vocab: int = 151936
    eps: float = 1e-6
    rope_theta: float = 1e6
    partial_rotary: float = 1.0
    block_size: int = 16
    group_size: int = 128
    weights: str = "w4g128"     # every Linear: "w4g128" (W4A16, group 128) or "w8" (int8 per output row)

    @classmethod
    def from_dict(cls, d: dict) -> "Qwen3Config":
        return cls(**{k: d[k] for k in cls.__dataclass_fields__ if k in d})

    @property
    def rot_dim(self) -> int:
        return int(self.head_dim * self.partial_rotary)


QWEN3_1P7B = Qwen3Config()
QWEN3_8B = Qwen3Config(layers=36, hidden=4096, heads=32, kv_heads=8, intermediate=12288)
QWEN3_8B_W8 = Qwen3Config(layers=36, hidden=4096, heads=32, kv_heads=8, intermediate=12288, weights="w8")


def rope_tables(theta: float, rot_dim: int, positions: int):
    """cos, sin fp32 [positions, rot_dim / 2] with torch's CPU operations in
    the order of _rope_inv_freq and _rope_cos_sin (layers.py:50-78)."""
    n_freq = rot_dim // 2
    inv = 1.0 / (theta ** (torch.arange(0, n_freq, dtype=torch.float32) / n_freq))
    pos = torch.arange(positions, dtype=torch.long).to(torch.float32).reshape(-1)
    freqs = pos.unsqueeze(1) * inv.unsqueeze(0)
    return torch.cos(freqs), torch.sin(freqs)


def _sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().contiguous().cpu().view(-1).view(torch.uint8).numpy().tobytes()).hexdigest()


@dataclass
class Qwen3Weights:
    """Device-resident weights: bf16 embedding and norms, and the linears with
    q/k/v and gate/up concatenated row-wise, either W4A16 g128 (qweight uint8
    [N, K/2], scales fp32 [N, K/128]) or int8 per output row (qweight int8
    [N, K], scales fp32 [N]; with bf16 activations the reference runs these
    through ekernel_linear_w8a16_bf16, linear.py:210-231)."""
    cfg: Qwen3Config
    embed: torch.Tensor
    layers: list
    norm: torch.Tensor
    lm_head: tuple
    quantized_sha: dict = field(default_factory=dict)

    @classmethod
    def synthetic(cls, cfg: Qwen3Config, seed: int, std: float = 0.02, device="cuda", hashes: bool = False):
        """Random-init weights ~N(0, std) (pilm_amd.synth_model, bit-identical on
        any device), every Linear quantized on the device with the reference's
        grouped int4 quantizer (ckernel.quantize_weight_i4_grouped_chunked) or,
        for cfg.weights "w8", its int8 per-row quantizer
        (ckernel.quantize_weight_i8_per_row_chunked)."""
        ids = SM.tensor_ids(cfg.layers)
        qsha = {}
        D, H, Hq, Hkv, I = cfg.head_dim, cfg.hidden, cfg.heads, cfg.kv_heads, cfg.intermediate

        def bf16(name, shape):
            return SM.normal_f32(seed, ids[name], shape, std, device=device).to(torch.bfloat16)

        def quant(name, out_f, in_f):
            w = SM.normal_f32(seed, ids[name], (out_f, in_f), std, device=device)
            if cfg.weights == "w8":
                q, s = ckernel.quantize_weight_i8_per_row_chunked(w, rows_per_chunk=8192)
            elif cfg.weights == "w4g128":
                q, s = ckernel.quantize_weight_i4_grouped_chunked(w, group_size=cfg.group_size, rows_per_chunk=8192)
            else:
                raise ValueError(f"unknown weight format {cfg.weights!r} (w4g128 or w8)")
            del w
            if hashes:
                qsha[name] = [_sha(q), _sha(s)]
            return q, s

        def cat(parts):
            return torch.cat([p[0] for p in parts]).contiguous(), torch.cat([p[1] for p in parts]).contiguous()

        layers = []
        for i in range(cfg.layers):
            p = f"layers.{i}."
            qkv = cat([quant(p + "self_attn.q_proj", 2 * Hq * D, H), quant(p + "self_attn.k_proj", Hkv * D, H),
                       quant(p + "self_attn.v_proj", Hkv * D, H)])
            gate_up = cat([quant(p + "mlp.gate", I, H), quant(p + "mlp.up", I, H)])
            layers.append({
                "in_norm": bf16(p + "input_layernorm", (H,)),
                "post_norm": bf16(p + "post_attention_layernorm", (H,)),
                "q_norm": bf16(p + "self_attn.q_norm", (D,)),
                "k_norm": bf16(p + "self_attn.k_norm", (D,)),
                "qkv": qkv,
                "o": quant(p + "self_attn.o_proj", H, Hq * D),
                "gate_up": gate_up,
                "down": quant(p + "mlp.down", H, I),
            })
        return cls(cfg, bf16("embed_tokens", (cfg.vocab, H)), layers, bf16("norm", (H,)),
                   quant("lm_head", cfg.vocab, H), qsha)

    def linear_bytes_per_token(self) -> int:
        """Weight + scale bytes the linears of one decode token read."""
        tot = sum(q.numel() + 4 * s.numel() for L in self.layers for (q, s) in (L["qkv"], L["o"], L["gate_up"],
                                                                                 L["down"]))
        return tot + self.lm_head[0].numel() + 4 * self.lm_head[1].numel()


def _vp(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else None)


class Qwen3Decoder:
    """One sequence's decode state: paged KV caches, rope tables, the device
    state word {pos0, cache_len, count} and the step buffers."""

    def __init__(self, weights: Qwen3Weights, max_positions: int, max_new_tokens: int = 1024,
                 max_rows: int | None = None, pool_blocks: int | None = None):
        self.w = w = weights
        self.cfg = c = weights.cfg
        dev = w.embed.device
        self.dev = dev
        self.lib = abi._load_lib()
        bs = c.block_size
        self.max_pos = max_positions
        self.nblocks = (max_positions + bs - 1) // bs          # blocks one sequence can use
        self.pool = pool_blocks or self.nblocks                  # blocks in each layer's cache
        kv_shape = (self.pool, bs, c.kv_heads, c.head_dim)
        self.k_cache = [torch.zeros(kv_shape, dtype=torch.bfloat16, device=dev) for _ in range(c.layers)]
        self.v_cache = [torch.zeros(kv_shape, dtype=torch.bfloat16, device=dev) for _ in range(c.layers)]
        # the reference's block manager hands out block ids; any assignment gives the same arithmetic
        self.block_ids = torch.arange(self.nblocks, dtype=torch.int32, device=dev)
        cos, sin = rope_tables(c.rope_theta, c.rot_dim, max_positions)
        self.cos, self.sin = cos.to(dev), sin.to(dev)
        S, H, D, Hq, I = max_rows or bs, c.hidden, c.head_dim, c.heads, c.intermediate
        self.max_rows = S
        e = dict(dtype=torch.bfloat16, device=dev)
        self.nqkv = w.layers[0]["qkv"][0].shape[0]
        self.x = torch.empty((S, H), **e)
        self.res = torch.empty((S, H), **e)
        self.h = torch.empty((S, H), **e)
        self.qkv = torch.empty((S, self.nqkv), **e)
        self.q = torch.empty((S, Hq, D), **e)
        self.attn = torch.empty((S, Hq * D), **e)
        self.o = torch.empty((S, H), **e)
        self.gu = torch.empty((S, 2 * I), **e)
        self.act = torch.empty((S, I), **e)
        self.mlp = torch.empty((S, H), **e)
        # residual rows of the fused decode step, alternating (a launch reads one, writes the other)
        self.res_pp = (torch.empty((1, H), **e), torch.empty((1, H), **e))
        self.logits = torch.empty((c.vocab,), **e)
        self.logits_rows = torch.empty((S, c.vocab), **e) if max_rows else None
        self.state = torch.zeros(4, dtype=torch.int32, device=dev)      # pos0, cache_len, count
        self.max_new = max_new_tokens
        self.tokens = torch.zeros(max_new_tokens, dtype=torch.int32, device=dev)
        self.next_id = torch.zeros(1, dtype=torch.int64, device=dev)
        self.graph = None
        self._descs = {}
        # the one-launch decode attention serves 64- and 128-wide heads, 1, 2 or 4 q heads per kv head
        self.fused_decode = c.head_dim in (64, 128) and c.heads // c.kv_heads in (1, 2, 4)
        # decode tokens: each GemmaRMSNorm inside the launch of the linear after it, SwiGLU inside gate_up
        # (the norm-fused GEMV is W4A16 g128)
        self.fused_norm = (self.fused_decode and c.weights == "w4g128" and c.hidden % 256 == 0
                           and c.hidden <= 16384)

    # ---------------------------------------------------------------- calls
    def _check(self, rc: int, name: str) -> None:
        if rc != 0:
            raise RuntimeError(f"{name} failed: rc={rc} ({abi.last_error()})")

    def _desc(self, key, maker):
        d = self._descs.get(key)
        if d is None:
            d = self._descs[key] = maker()
        return d

    def _linear(self, x, wq, out, m):
        q, s = wq
        d = self._desc(("lin", m, q.shape[0], x.shape[1]),
                       lambda: abi.EkernelLinearW8A32Desc(m, q.shape[0], x.shape[1]))
        if q.dtype == torch.int8:
            self._check(self.lib.ekernel_linear_w8a16_bf16(ctypes.byref(d), _vp(x), _vp(q), _vp(s), _vp(out), 6),
                        "ekernel_linear_w8a16_bf16")
        else:
            self._check(self.lib.ekernel_linear_w4a16g128_bf16(ctypes.byref(d), _vp(x), _vp(q), _vp(s), _vp(out),
                                                               6), "ekernel_linear_w4a16g128_bf16")

    def _norm(self, x, res, weight, out, res_out, m):
        d = self._desc(("norm", m), lambda: abi.EkernelRmsnormDesc(m, self.cfg.hidden, self.cfg.eps))
        self._check(self.lib.ekernel_rmsnorm_gemma_bf16(ctypes.byref(d), _vp(x), _vp(res), _vp(weight), _vp(out),
                                                        _vp(res_out)), "ekernel_rmsnorm_gemma_bf16")

    def _norm_linear(self, x, res, weight, res_out, wq, out, swiglu):
        q, s = wq
        d = self._desc(("normlin", q.shape[0], swiglu),
                       lambda: abi.EkernelNormLinearDesc(1, q.shape[0], self.cfg.hidden, self.cfg.eps, int(swiglu)))
        self._check(self.lib.ekernel_rmsnorm_linear_w4a16g128_bf16(ctypes.byref(d), _vp(x), _vp(res), _vp(weight),
                                                                  _vp(res_out), _vp(q), _vp(s), _vp(out)),
                    "ekernel_rmsnorm_linear_w4a16g128_bf16")

    def _forward_decode(self):
        """One decode token (self.x[0]) with five launches per layer: input
        norm + qkv, attention, o, post-attention norm + gate_up + SwiGLU,
        down; the residual rows alternate between two buffers."""
        c, L = self.cfg, self.lib
        D, Hq, Hkv = c.head_dim, c.heads, c.kv_heads
        qkv_p = self.qkv.data_ptr()
        k_off, v_off = 2 * Hq * D * 2, (2 * Hq * D + Hkv * D) * 2
        rope = self._desc(("rope", 1), lambda: abi.EkernelQkRopeDesc(
            1, Hq, Hkv, D, c.rot_dim, self.nqkv, self.nqkv, 0, self.max_pos, c.block_size, self.pool,
            self.block_ids.numel(), c.eps))
        r0, r1 = self.res_pp
        x1, res_prev = self.x[:1], None
        for li, Lw in enumerate(self.w.layers):
            if li == 0:
                self._norm_linear(x1, None, Lw["in_norm"], None, Lw["qkv"], self.qkv[:1], False)
                res_in = x1
            else:
                self._norm_linear(self.mlp[:1], res_prev, Lw["in_norm"], r0, Lw["qkv"], self.qkv[:1], False)
                res_in = r0
            self._check(L.ekernel_decode_attention_bf16(
                ctypes.byref(rope), ctypes.c_void_p(qkv_p), ctypes.c_void_p(qkv_p + k_off),
                ctypes.c_void_p(qkv_p + v_off), _vp(Lw["q_norm"]), _vp(Lw["k_norm"]), _vp(self.cos), _vp(self.sin),
                _vp(self.state), _vp(self.k_cache[li]), _vp(self.v_cache[li]), _vp(self.block_ids),
                _vp(self.attn)), "ekernel_decode_attention_bf16")
            self._linear(self.attn[:1], Lw["o"], self.o[:1], 1)
            self._norm_linear(self.o[:1], res_in, Lw["post_norm"], r1, Lw["gate_up"], self.act[:1], True)
            self._linear(self.act[:1], Lw["down"], self.mlp[:1], 1)
            res_prev = r1
        self._norm(self.mlp[:1], res_prev, self.w.norm, self.h, None, 1)
        self._linear(self.h[:1], self.w.lm_head, self.logits.view(1, -1), 1)
        self._check(L.ekernel_greedy_step_bf16(_vp(self.logits), c.vocab, _vp(self.state), _vp(self.tokens),
                                               self.max_new, _vp(self.next_id)), "ekernel_greedy_step_bf16")

    def _forward(self, m: int, with_logits: bool, groups=None):
        """The model over the m tokens in self.x.  groups None: one sequence at
        the positions the state word names (graph-capturable); with_logits:
        final norm + lm_head of the last token and the greedy step.  groups:
        [(row0, rows, pos0, block table[, sequence])] -- several sequences'
        rows in one batch, positions from the host; the linears take all m
        rows at once and with_logits gives the logits of every row
        (self.logits_rows).  With the sequence index (the row of its table in
        self.tables_all) rope and attention take every sequence's rows in one
        launch each; otherwise one pair of launches per sequence."""
        c, L = self.cfg, self.lib
        D, Hq, Hkv, I = c.head_dim, c.heads, c.kv_heads, c.intermediate
        qkv_p = self.qkv.data_ptr()
        k_off, v_off = 2 * Hq * D * 2, (2 * Hq * D + Hkv * D) * 2
        batch = None
        if groups is None:
            groups_run = [(0, m, None, self.block_ids)]
        else:
            groups_run = [g[:4] for g in groups]
            tables_all = getattr(self, "tables_all", None)
            if tables_all is not None and len(groups[0]) == 5 and m <= 128:
                n_tables = len(self.tables)
                per = tables_all.numel() // n_tables
                seqs = (abi.EkernelBatchSeq * len(groups))(
                    *[abi.EkernelBatchSeq(r0, n, pos0, sq) for (r0, n, pos0, _, sq) in groups])
                rope_b = abi.EkernelQkRopeDesc(m, Hq, Hkv, D, c.rot_dim, self.nqkv, self.nqkv, 0, self.max_pos,
                                               c.block_size, self.pool, per, c.eps)
                att_b = abi.EkernelAttentionExactDesc(m, Hq, Hkv, D, 0, c.block_size, self.pool, per, self.nqkv,
                                                      2 * D)
                batch = (seqs, len(groups), rope_b, att_b, tables_all, n_tables)
        res_in = None
        for li, Lw in enumerate(self.w.layers):
            if li == 0:
                self._norm(self.x, None, Lw["in_norm"], self.h, None, m)
                res_in = self.x
            else:
                self._norm(self.mlp, self.res, Lw["in_norm"], self.h, self.res, m)
                res_in = self.res
            self._linear(self.h, Lw["qkv"], self.qkv, m)
            if batch is not None:
                # every sequence's rows in one rope launch and one attention launch
                seqs, nseq, rope_b, att_b, tables_all, n_tables = batch
                q_p = self.q.data_ptr()
                self._check(L.ekernel_qk_norm_rope_batch_bf16(
                    ctypes.byref(rope_b), seqs, nseq, n_tables, ctypes.c_void_p(qkv_p), ctypes.c_void_p(qkv_p + k_off),
                    ctypes.c_void_p(qkv_p + v_off), _vp(Lw["q_norm"]), _vp(Lw["k_norm"]), _vp(self.cos),
                    _vp(self.sin), ctypes.c_void_p(q_p), _vp(self.k_cache[li]), _vp(self.v_cache[li]),
                    _vp(tables_all)), "ekernel_qk_norm_rope_batch_bf16")
                self._check(L.ekernel_attention_exact_batch_bf16(
                    ctypes.byref(att_b), seqs, nseq, n_tables, ctypes.c_void_p(q_p), _vp(self.k_cache[li]),
                    _vp(self.v_cache[li]), _vp(tables_all), ctypes.c_void_p(qkv_p + D * 2),
                    _vp(self.attn)), "ekernel_attention_exact_batch_bf16")
            else:
                for (r0, n, pos0, table) in groups_run:
                    def mk_rope():
                        return abi.EkernelQkRopeDesc(n, Hq, Hkv, D, c.rot_dim, self.nqkv, self.nqkv, pos0 or 0,
                                                     self.max_pos, c.block_size, self.pool, table.numel(), c.eps)

                    def mk_att():
                        return abi.EkernelAttentionExactDesc(n, Hq, Hkv, D, (pos0 or 0) + n, c.block_size, self.pool,
                                                             table.numel(), self.nqkv, 2 * D)
                    # one sequence's descriptors are reused; batch positions change every step
                    rope = self._desc(("rope", n), mk_rope) if pos0 is None else mk_rope()
                    att = self._desc(("attn", n), mk_att) if pos0 is None else mk_att()
                    step = self.state if pos0 is None else None
                    rp = qkv_p + r0 * self.nqkv * 2
                    if n == 1 and self.fused_decode:
                        # one decode row: norm, rope, cache write and attention in one launch
                        self._check(L.ekernel_decode_attention_bf16(
                            ctypes.byref(rope), ctypes.c_void_p(rp), ctypes.c_void_p(rp + k_off),
                            ctypes.c_void_p(rp + v_off), _vp(Lw["q_norm"]), _vp(Lw["k_norm"]), _vp(self.cos),
                            _vp(self.sin), _vp(step), _vp(self.k_cache[li]), _vp(self.v_cache[li]), _vp(table),
                            ctypes.c_void_p(self.attn.data_ptr() + r0 * Hq * D * 2)), "ekernel_decode_attention_bf16")
                        continue
                    self._check(L.ekernel_qk_norm_rope_bf16(
                        ctypes.byref(rope), ctypes.c_void_p(rp), ctypes.c_void_p(rp + k_off),
                        ctypes.c_void_p(rp + v_off), _vp(Lw["q_norm"]), _vp(Lw["k_norm"]), _vp(self.cos),
                        _vp(self.sin), _vp(step),
                        ctypes.c_void_p(self.q.data_ptr() + r0 * Hq * D * 2), _vp(self.k_cache[li]),
                        _vp(self.v_cache[li]), _vp(table)), "ekernel_qk_norm_rope_bf16")
                    self._check(L.ekernel_attention_exact_bf16(
                        ctypes.byref(att), ctypes.c_void_p(self.q.data_ptr() + r0 * Hq * D * 2), _vp(self.k_cache[li]),
                        _vp(self.v_cache[li]), _vp(table), ctypes.c_void_p(rp + D * 2), _vp(step),
                        ctypes.c_void_p(self.attn.data_ptr() + r0 * Hq * D * 2)), "ekernel_attention_exact_bf16")
            self._linear(self.attn, Lw["o"], self.o, m)
            self._norm(self.o, res_in, Lw["post_norm"], self.h, self.res, m)
            self._linear(self.h, Lw["gate_up"], self.gu, m)
            gp = self.gu.data_ptr()
            self._check(L.ekernel_silu_mul_bf16(ctypes.c_void_p(gp), ctypes.c_void_p(gp + I * 2), m, I, 2 * I,
                                                _vp(self.act)), "ekernel_silu_mul_bf16")
            self._linear(self.act, Lw["down"], self.mlp, m)
        if with_logits and groups is None:
            last = m - 1
            self._norm(self.mlp[last:m], self.res[last:m], self.w.norm, self.h, None, 1)
            self._linear(self.h[:1], self.w.lm_head, self.logits.view(1, -1), 1)
            self._check(L.ekernel_greedy_step_bf16(_vp(self.logits), c.vocab, _vp(self.state), _vp(self.tokens),
                                                   self.max_new, _vp(self.next_id)), "ekernel_greedy_step_bf16")
        elif with_logits:
            self._norm(self.mlp, self.res, self.w.norm, self.h, None, m)
            self._linear(self.h, self.w.lm_head, self.logits_rows, m)

    def _bind(self):
        abi.set_stream(torch.cuda.current_stream(self.dev).cuda_stream)

    # ---------------------------------------------------------------- public
    def prefill(self, prompt: list) -> None:
        """Prompt tokens in the engine's chunks (each within one KV block);
        the last chunk's logits give the first generated token."""
        c = self.cfg
        if len(prompt) + 1 > self.max_pos:
            raise ValueError(f"prompt of {len(prompt)} tokens exceeds {self.max_pos} positions")
        self._bind()
        ids = torch.tensor(prompt, dtype=torch.int64, device=self.dev)
        pos = 0
        while pos < len(prompt):
            n = min(len(prompt) - pos, c.block_size - pos % c.block_size)
            self.state.copy_(torch.tensor([pos, pos + n, 0, 0], dtype=torch.int32))
            torch.index_select(self.w.embed, 0, ids[pos:pos + n], out=self.x[:n])
            self._forward(n, with_logits=pos + n == len(prompt))
            pos += n

    def decode_step(self) -> None:
        """One token: embedding of the last generated id, the model, lm_head,
        argmax; advances the state word."""
        torch.index_select(self.w.embed, 0, self.next_id, out=self.x[:1])
        if self.fused_norm:
            self._forward_decode()
        else:
            self._forward(1, with_logits=True)

    def capture(self) -> None:
        """Capture decode_step into a HIP graph (the state word makes each
        replay the next position).  One eager step first sizes the library's
        per-device scratch (split-K sums and tickets), which must not be
        allocated while a graph is being captured; the state, the next id and
        the token list are restored after it, and the first replay recomputes
        that step (its cache rows come out the same)."""
        saved = (self.state.clone(), self.next_id.clone(), self.tokens.clone())
        self._bind()
        self.decode_step()
        torch.cuda.synchronize(self.dev)
        self.state.copy_(saved[0])
        self.next_id.copy_(saved[1])
        self.tokens.copy_(saved[2])
        s = torch.cuda.Stream(self.dev)
        s.wait_stream(torch.cuda.current_stream(self.dev))
        torch.cuda.synchronize(self.dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s, capture_error_mode="relaxed"):
            self._bind()
            self.decode_step()
        torch.cuda.synchronize(self.dev)
        self._bind()
        self.graph = g

    def generate(self, prompt: list, n_new: int, graph: bool = True, on_logits=None) -> list:
        """Greedy tokens after the prompt (src/engine.py:383-659 with
        temperature 0, top_k 0).  on_logits(i, logits) sees the bf16 logits
        each token i was chosen from (eager steps only)."""
        if n_new > self.max_new or len(prompt) + n_new > self.max_pos:
            raise ValueError("sequence longer than the decoder was sized for")
        if on_logits is not None:
            graph = False
        self.prefill(prompt)
        if on_logits is not None:
            on_logits(0, self.logits)
        if graph and n_new > 1:
            if self.graph is None:
                self.capture()        # records the step; nothing runs until a replay
            for _ in range(n_new - 1):
                self.graph.replay()
        else:
            self._bind()
            for i in range(1, n_new):
                self.decode_step()
                if on_logits is not None:
                    on_logits(i, self.logits)
        torch.cuda.synchronize(self.dev)
        return self.tokens[:n_new].tolist()


def accept_drafts(logits_rows: torch.Tensor, drafts: list) -> tuple:
    """Greedy MTP verification of one sequence (src/engine.py:467-545): row i
    of the logits (rows 0 .. len(drafts)) is what the model predicts after the
    sequence's last token and drafts[:i]; drafts are accepted while each
    equals the argmax of the row before it; the first mismatch's argmax, or
    when all are accepted the argmax of the last row, is the next token.
    Returns (accepted drafts, next token).  Argmax as torch.argmax on the
    fp32 copy: the first index of the largest value."""
    return accept_draft_ids(torch.argmax(logits_rows.to(torch.float32), dim=-1).tolist(), drafts)


def accept_draft_ids(ids: list, drafts: list) -> tuple:
    """accept_drafts on the rows' argmax ids already taken."""
    acc = []
    for i, d in enumerate(drafts):
        if ids[i] != int(d):
            return acc, ids[i]
        acc.append(int(d))
    return acc, ids[len(drafts)]


class Qwen3Batch(Qwen3Decoder):
    """Several sequences decoding together (continuous batching,
    src/runtime/scheduler/scheduler.py:70-178): one paged KV pool per layer,
    one block table per sequence, and steps that pass every sequence's rows
    as one M to the linears -- an MTP verify step of 16 sequences x (1 + 4
    drafts) is one M = 80 call per linear.  With exact (the default) the
    linears run on the bit-exact kernels at every M (the matrix-core
    threshold is lowered to none for the step), so each sequence's logits
    are bit-identical to its own per-sequence run, as the reference verifies
    each sequence by itself (src/engine.py:416-459).  exact=False leaves the
    library's threshold: batches of 64 rows or more go to the matrix cores
    (outputs within their 1e-2 tolerance, not bit-identical; an argmax at a
    near tie can then differ from the reference's)."""

    def __init__(self, weights: Qwen3Weights, n_seqs: int, max_positions: int, max_rows: int = 96,
                 exact: bool = True):
        bs = weights.cfg.block_size
        per_seq = (max_positions + bs - 1) // bs
        super().__init__(weights, max_positions, max_new_tokens=1, max_rows=max_rows,
                         pool_blocks=per_seq * n_seqs)
        self.tables_all = torch.arange(n_seqs * per_seq, dtype=torch.int32, device=self.dev)
        self.tables = [self.tables_all[i * per_seq:(i + 1) * per_seq] for i in range(n_seqs)]
        self.cache_len = [0] * n_seqs
        self.exact = exact

    def _run(self, groups_tokens, with_logits: bool):
        rows = sum(len(t) for _, t in groups_tokens)
        if rows > self.max_rows:
            raise ValueError(f"{rows} rows exceed the batch buffers ({self.max_rows})")
        ids = torch.tensor([t for _, toks in groups_tokens for t in toks], dtype=torch.int64, device=self.dev)
        torch.index_select(self.w.embed, 0, ids, out=self.x[:rows])
        groups, r0 = [], 0
        for seq, toks in groups_tokens:
            pos0 = self.cache_len[seq]
            if pos0 + len(toks) > self.max_pos:
                raise ValueError(f"sequence {seq} would exceed {self.max_pos} positions")
            groups.append((r0, len(toks), pos0, self.tables[seq], seq))
            r0 += len(toks)
        if not self.exact:
            self._bind()
            self._forward(rows, with_logits, groups=groups)
            return rows
        prev = abi.matrix_core_min_rows()
        abi.set_matrix_core_min_rows(0)          # 0: exact kernels at every M
        try:
            self._bind()
            self._forward(rows, with_logits, groups=groups)
        finally:
            abi.set_matrix_core_min_rows(prev)
        return rows

    def prefill_seq(self, seq: int, prompt: list) -> int:
        """One sequence's prompt in the engine's block-aligned chunks; returns
        the greedy first token."""
        bs = self.cfg.block_size
        self.cache_len[seq] = 0
        pos = 0
        while pos < len(prompt):
            n = min(len(prompt) - pos, bs - pos % bs)
            rows = self._run([(seq, prompt[pos:pos + n])], with_logits=pos + n == len(prompt))
            self.cache_len[seq] += n
            pos += n
        return int(torch.argmax(self.logits_rows[rows - 1].to(torch.float32)).item())

    def prefill_seqs(self, seqs: list, prompts: list) -> list:
        """Several sequences' prompts together: each step packs the next
        block-aligned chunk of every unfinished sequence into one batch of at
        most max_rows rows.  Returns each sequence's greedy first token."""
        bs = self.cfg.block_size
        pos = {s: 0 for s in seqs}
        for s in seqs:
            self.cache_len[s] = 0
        first = {}
        while len(first) < len(seqs):
            groups, rows, final = [], 0, []
            for s, p in zip(seqs, prompts):
                if s in first:
                    continue
                n = min(len(p) - pos[s], bs - pos[s] % bs)
                if rows + n > self.max_rows:
                    break
                groups.append((s, p[pos[s]:pos[s] + n]))
                if pos[s] + n == len(p):
                    final.append((s, rows + n - 1))
                rows += n
            if not groups:
                raise ValueError(f"a chunk of {bs} rows exceeds the batch buffers ({self.max_rows})")
            self._run(groups, with_logits=bool(final))
            for s, toks in groups:
                self.cache_len[s] += len(toks)
                pos[s] += len(toks)
            for s, r in final:
                first[s] = int(torch.argmax(self.logits_rows[r].to(torch.float32)).item())
        return [first[s] for s in seqs]

    def verify(self, last_tokens: list, drafts: list) -> list:
        """One verify step for every sequence: sequence i feeds
        [last_tokens[i]] + drafts[i] (its positions follow its cache); all rows
        go through the model as one batch; returns [(accepted, next token)]
        per sequence and advances each cache past the accepted tokens."""
        groups = [(i, [int(last_tokens[i])] + [int(d) for d in drafts[i]]) for i in range(len(drafts))]
        rows = self._run(groups, with_logits=True)
        # every row's argmax in one pass and one copy to the host
        ids = torch.argmax(self.logits_rows[:rows].to(torch.float32), dim=-1).tolist()
        out, r0 = [], 0
        for (i, toks) in groups:
            acc, nxt = accept_draft_ids(ids[r0:r0 + len(toks)], drafts[i])
            out.append((acc, nxt))
            self.cache_len[i] += 1 + len(acc)
            r0 += len(toks)
        return out
