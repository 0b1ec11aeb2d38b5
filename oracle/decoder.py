"""Python face of the decoder-step oracle -- TEST INFRASTRUCTURE ONLY.

Loads oracle/_build/liboracle_decoder.so (oracle/decoder.c: the torch steps
of piLM's Qwen3 decoder layer with torch's CPU roundings) and assembles the
whole decoder from it, the linear oracle (oracle.c) and the numpy quantizer
restatement (oracle.py).  `OracleDecoder` replays piLM's Engine.generate
schedule (src/engine.py:383-459: prefill in block-aligned chunks of at most
one block, then one token per step, greedy argmax) so its tokens and
per-step logits can be compared with the fixtures the reference itself
wrote (tests/golden/decode_*.json).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module.
"""
from __future__ import annotations

import ctypes
import hashlib
from pathlib import Path

import numpy as np

from oracle import oracle as O

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle_decoder.so"

_P = ctypes.c_void_p
_S = ctypes.c_size_t
_F = ctypes.c_float
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            O.build(ref=False)
        L = ctypes.CDLL(str(LIB))
        L.oracle_sleef_expf.argtypes = [_F]
        L.oracle_sleef_expf.restype = _F
        L.oracle_sleef_expf_n.argtypes = [_P, _P, _S]
        L.oracle_torch_sum.argtypes = [_P, _S]
        L.oracle_torch_sum.restype = _F
        L.oracle_rmsnorm_gemma_bf16.argtypes = [_S, _S, _F, _P, _P, _P, _P, _P]
        L.oracle_qk_norm_rope_bf16.argtypes = [_S, _S, _S, _S, _S, _S, _S, _S, _F] + [_P] * 11 + [_S]
        L.oracle_attention_exact_bf16.argtypes = [_S, _S, _S, _S, _S, _S, _P, _P, _P, _P, _P, _S, _S, _P]
        L.oracle_silu_mul_bf16.argtypes = [_P, _P, _S, _S, _S, _P]
        L.oracle_sigmoid_bf16.argtypes = [_P, _P, _S]
        L.oracle_silu_bf16.argtypes = [_P, _P, _S]
        L.oracle_softmax_f32.argtypes = [_P, _P, _S, _S]
        L.oracle_argmax_bf16.argtypes = [_P, _S]
        L.oracle_argmax_bf16.restype = _S
        _lib = L
    return _lib


def _p(a) -> int | None:
    return None if a is None else a.ctypes.data


def _u16(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint16)


def sleef_expf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().oracle_sleef_expf_n(_p(x), _p(out), x.size)
    return out


def torch_sum(x: np.ndarray) -> np.float32:
    x = np.ascontiguousarray(x, np.float32)
    return np.float32(lib().oracle_torch_sum(_p(x), x.size))


def softmax_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().oracle_softmax_f32(_p(x), _p(out), x.shape[0], x.shape[1])
    return out


def sigmoid_bf16(x: np.ndarray) -> np.ndarray:
    x = _u16(x)
    out = np.empty_like(x)
    lib().oracle_sigmoid_bf16(_p(x), _p(out), x.size)
    return out


def silu_bf16(x: np.ndarray) -> np.ndarray:
    x = _u16(x)
    out = np.empty_like(x)
    lib().oracle_silu_bf16(_p(x), _p(out), x.size)
    return out


def rmsnorm_gemma_bf16(x, residual, weight, eps: float):
    """(out, residual_out) for bf16 bit arrays [rows, n]; residual may be None."""
    x = _u16(x)
    rows, n = x.shape
    res = None if residual is None else _u16(residual)
    out = np.empty_like(x)
    res_out = None if res is None else np.empty_like(x)
    lib().oracle_rmsnorm_gemma_bf16(rows, n, eps, _p(x), _p(res), _p(_u16(weight)), _p(out), _p(res_out))
    return out, res_out


def qk_norm_rope_bf16(qg, k, v, q_w, k_w, cos_t, sin_t, pos0, k_cache, v_cache, block_ids, *, n_heads, n_kv_heads,
                      head_dim, rot_dim, eps, block_size):
    """q_out [S, H, D]; writes k / v rows into the caches (numpy, in place)."""
    qg, k, v = _u16(qg), _u16(k), _u16(v)
    S = qg.shape[0]
    q_out = np.empty((S, n_heads, head_dim), np.uint16)
    cos_t = np.ascontiguousarray(cos_t, np.float32)
    sin_t = np.ascontiguousarray(sin_t, np.float32)
    bids = np.ascontiguousarray(block_ids, np.int32)
    lib().oracle_qk_norm_rope_bf16(S, n_heads, n_kv_heads, head_dim, rot_dim, qg.shape[1], k.shape[1], pos0, eps,
                                   _p(qg), _p(k), _p(v), _p(_u16(q_w)), _p(_u16(k_w)), _p(cos_t), _p(sin_t),
                                   _p(q_out), _p(k_cache), _p(v_cache), _p(bids), block_size)
    return q_out


def attention_exact_bf16(q, k_cache, v_cache, block_ids, cache_len, gate=None, gate_row_stride=0,
                         gate_head_stride=0, *, block_size):
    """out [S, H * D] for q [S, H, D] over caches [blocks, bs, Hkv, D]."""
    q = _u16(q)
    S, H, D = q.shape
    Hkv = k_cache.shape[2]
    out = np.empty((S, H * D), np.uint16)
    bids = np.ascontiguousarray(block_ids, np.int32)
    g = None if gate is None else _u16(gate)
    lib().oracle_attention_exact_bf16(S, H, Hkv, D, cache_len, block_size, _p(bids), _p(q), _p(k_cache),
                                      _p(v_cache), _p(g), gate_row_stride, gate_head_stride, _p(out))
    return out


def silu_mul_bf16(gate, up, rows, n, in_stride):
    """gate / up: contiguous bf16 arrays holding rows of in_stride elements."""
    gate, up = _u16(gate), _u16(up)
    if gate.size < (rows - 1) * in_stride + n or up.size < (rows - 1) * in_stride + n:
        raise ValueError("gate / up smaller than rows x in_stride")
    out = np.empty((rows, n), np.uint16)
    lib().oracle_silu_mul_bf16(_p(_u16(gate)), _p(_u16(up)), rows, n, in_stride, _p(out))
    return out


def argmax_bf16(x) -> int:
    x = _u16(x)
    return int(lib().oracle_argmax_bf16(_p(x), x.size))


def rope_tables(theta: float, rot_dim: int, positions: int):
    """(cos, sin) fp32 [positions, rot_dim / 2] computed with torch's CPU
    operations in the order of _rope_inv_freq / _rope_cos_sin (layers.py:50-78)."""
    import torch
    n_freq = rot_dim // 2
    inv = 1.0 / (theta ** (torch.arange(0, n_freq, dtype=torch.float32) / n_freq))
    freqs = torch.arange(positions, dtype=torch.long).to(torch.float32).reshape(-1).unsqueeze(1) * inv.unsqueeze(0)
    return torch.cos(freqs).numpy(), torch.sin(freqs).numpy()


def sha_u16(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).view(np.uint8).tobytes()).hexdigest()


class OracleDecoder:
    """piLM's Qwen3Model (all layers full attention, every Linear W4A16 g128,
    or with cfg["weights"] == "w8" int8 per output row run as W8A16 on the
    bf16 activations, linear.py:210-231) evaluated with the oracle, on the
    fixture's seeded weights."""

    def __init__(self, cfg: dict):
        import torch
        from pilm_amd import synth_model as SM
        self.cfg = c = cfg
        self.w8 = c.get("weights", "w4g128") == "w8"
        L, H, V = c["layers"], c["hidden"], c["vocab"]
        ids = SM.tensor_ids(L)
        seed, std = c["seed"], c["std"]
        self.qsha = {}

        def bf16(name, shape):
            t = SM.normal_f32(seed, ids[name], shape, std).to(torch.bfloat16)
            return t.view(torch.int16).numpy().view(np.uint16).copy()

        def quant(name, out_f, in_f):
            w = SM.normal_f32(seed, ids[name], (out_f, in_f), std).numpy()
            if self.w8:
                q, s = O.quantize_weight_i8_per_row(w)
            else:
                q, s = O.quantize_weight_i4_grouped(w, c["group_size"])
            self.qsha[name] = [hashlib.sha256(q.tobytes()).hexdigest(), hashlib.sha256(s.tobytes()).hexdigest()]
            return q, s

        D, Hq, Hkv, I = c["head_dim"], c["heads"], c["kv_heads"], c["intermediate"]
        self.embed = bf16("embed_tokens", (V, H))
        self.layers = []
        for i in range(L):
            p = f"layers.{i}."
            self.layers.append({
                "in_norm": bf16(p + "input_layernorm", (H,)),
                "post_norm": bf16(p + "post_attention_layernorm", (H,)),
                "q_norm": bf16(p + "self_attn.q_norm", (D,)),
                "k_norm": bf16(p + "self_attn.k_norm", (D,)),
                "q": quant(p + "self_attn.q_proj", 2 * Hq * D, H),
                "k": quant(p + "self_attn.k_proj", Hkv * D, H),
                "v": quant(p + "self_attn.v_proj", Hkv * D, H),
                "o": quant(p + "self_attn.o_proj", H, Hq * D),
                "gate": quant(p + "mlp.gate", I, H),
                "up": quant(p + "mlp.up", I, H),
                "down": quant(p + "mlp.down", H, I),
            })
        self.norm = bf16("norm", (H,))
        self.lm_head = quant("lm_head", V, H)
        self.rot = int(D * c["partial_rotary"])
        self.max_pos = c["prompt"] + c["new_tokens"] + 1
        self.cos, self.sin = rope_tables(c["rope_theta"], self.rot, self.max_pos)
        bs = c["block_size"]
        self.nblocks = (self.max_pos + bs - 1) // bs
        self.block_ids = np.arange(self.nblocks, dtype=np.int32)
        self.k_cache = [np.zeros((self.nblocks, bs, Hkv, D), np.uint16) for _ in range(L)]
        self.v_cache = [np.zeros((self.nblocks, bs, Hkv, D), np.uint16) for _ in range(L)]

    def _lin(self, x, qs):
        q, s = qs
        if self.w8:
            return O.linear_w8a16_bf16(x, q, s)
        return O.linear_w4a16g_bf16(x, q, s, self.cfg["group_size"])

    def forward(self, ids, pos0, all_rows=False):
        """bf16 logits of the last of the S tokens at positions pos0.., or of
        every row (all_rows: the speculative verify of src/engine.py:462-476,
        lm_head over the whole normed output)."""
        c = self.cfg
        D, Hq, Hkv, I, eps = c["head_dim"], c["heads"], c["kv_heads"], c["intermediate"], c["eps"]
        S = len(ids)
        x = self.embed[np.asarray(ids)]
        res = None
        h = None
        for li, Lw in enumerate(self.layers):
            if res is None:
                h, _ = rmsnorm_gemma_bf16(x, None, Lw["in_norm"], eps)
                res = x
            else:
                h, res = rmsnorm_gemma_bf16(x, res, Lw["in_norm"], eps)
            qg = self._lin(h, Lw["q"])
            k = self._lin(h, Lw["k"])
            v = self._lin(h, Lw["v"])
            q = qk_norm_rope_bf16(qg, k, v, Lw["q_norm"], Lw["k_norm"], self.cos, self.sin, pos0,
                                  self.k_cache[li], self.v_cache[li], self.block_ids, n_heads=Hq,
                                  n_kv_heads=Hkv, head_dim=D, rot_dim=self.rot, eps=eps,
                                  block_size=c["block_size"])
            gate = qg.reshape(-1)[D:]          # gate of (s, h) at s * 2HD + h * 2D + D
            attn = attention_exact_bf16(q, self.k_cache[li], self.v_cache[li], self.block_ids, pos0 + S,
                                        gate, 2 * Hq * D, 2 * D, block_size=c["block_size"])
            o = self._lin(attn, Lw["o"])
            h, res = rmsnorm_gemma_bf16(o, res, Lw["post_norm"], eps)
            g = self._lin(h, Lw["gate"])
            u = self._lin(h, Lw["up"])
            act = silu_mul_bf16(g, u, S, I, I)
            x = self._lin(act, Lw["down"])
        if all_rows:
            hN, _ = rmsnorm_gemma_bf16(x, res, self.norm, eps)
            return self._lin(hN, self.lm_head)
        hN, _ = rmsnorm_gemma_bf16(x[-1:], res[-1:], self.norm, eps)
        return self._lin(hN, self.lm_head)[0]

    def generate(self, prompt, n_new, on_logits=None):
        """Greedy tokens after the prompt, with the engine's chunked prefill."""
        bs = self.cfg["block_size"]
        pos = 0
        tokens = []
        while pos < len(prompt):
            n = min(len(prompt) - pos, bs - pos % bs)
            logits = self.forward(prompt[pos:pos + n], pos)
            pos += n
        while True:
            t = argmax_bf16(logits)
            if on_logits:
                on_logits(len(tokens), logits)
            tokens.append(t)
            if len(tokens) == n_new:
                return tokens
            logits = self.forward([t], pos)
            pos += 1
