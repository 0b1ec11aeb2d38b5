#!/usr/bin/env python3
"""Writes tests/golden/verify_qwen3_1p7b.json: a 16-sequence speculative
(MTP) decode of Qwen3-1.7B W4A16 g128 as the reference's engine verifies it
(src/engine.py:416-545), computed with the oracle (oracle/decoder.py).

Every sequence starts from the 128-token prompt of decode_qwen3_1p7b.json
(the reference's own greedy decode).  At each step sequence i offers 4
drafts: the reference's greedy tokens that follow what it has emitted, draft
(i + step) % 5 replaced by a wrong token (4 = none).  The verify call runs
the model over [last token] + drafts (S = 5 rows, lm_head on every row) and
accepts drafts while each equals the argmax of the row before it.

A verify row is not always bit-identical to the single-row decode step at
the same position: torch's bf16 product of the attention weights with V
(attention.py:133-137) assigns positions to its four partial sums by their
index within the masked row, so the masked zeros at the end of an S = 5
row's weights move the last unmasked positions onto other partial sums.  The
resulting one-ulp differences can flip a near tie, so a speculative decode
may leave the plain greedy tokens; the fixture records what the verify rows
give.  Recorded per sequence and step: the drafts, accepted drafts, next
token and the sha256 of the five rows' bf16 logits.

One process (the oracle's linears use every core through OpenMP): the
prompt is prefilled once and each sequence starts from a copy of that cache.
About 30 minutes on 8 cores.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

N_SEQ, STEPS, DRAFTS = 16, 8, 4


def drafts_for(ref, n, i, step, vocab):
    d = list(ref[n:n + DRAFTS])
    bad = (i + step) % (DRAFTS + 1)
    if bad < DRAFTS:
        d[bad] = (d[bad] + 1 + i + step) % vocab
    return d


def run_sequence(od, snap, i, ref, prompt_len, vocab):
    import numpy as np
    from oracle import decoder as OD
    for li in range(len(od.k_cache)):
        np.copyto(od.k_cache[li], snap[0][li])
        np.copyto(od.v_cache[li], snap[1][li])
    emitted = [snap[2]]
    steps = []
    for step in range(STEPS):
        n = len(emitted)
        d = drafts_for(ref, n, i, step, vocab)
        rows = od.forward([emitted[-1]] + d, prompt_len + n - 1, all_rows=True)
        ids = [OD.argmax_bf16(r) for r in rows]
        acc = []
        for k, t in enumerate(d):
            if ids[k] != t:
                break
            acc.append(t)
        nxt = ids[len(acc)]
        emitted += acc + [nxt]
        steps.append({"drafts": d, "accepted": acc, "next": nxt,
                      "rows_sha": hashlib.sha256(np.ascontiguousarray(rows).tobytes()).hexdigest()})
        print(f"sequence {i} step {step}: accepted {len(acc)}", flush=True)
    return {"sequence": i, "first": snap[2], "steps": steps, "emitted": emitted}


def main():
    from oracle import decoder as OD
    fx = json.loads((HERE / "decode_qwen3_1p7b.json").read_text())
    cfg, ref, prompt = fx["config"], fx["tokens"], fx["prompt"]
    od = OD.OracleDecoder(cfg)
    bs, pos = cfg["block_size"], 0
    while pos < len(prompt):
        n = min(len(prompt) - pos, bs - pos % bs)
        logits = od.forward(prompt[pos:pos + n], pos)
        pos += n
    print("prompt prefilled", flush=True)
    snap = ([k.copy() for k in od.k_cache], [v.copy() for v in od.v_cache], OD.argmax_bf16(logits))
    seqs = [run_sequence(od, snap, i, ref, len(prompt), cfg["vocab"]) for i in range(N_SEQ)]
    diverged = [s["sequence"] for s in seqs if s["emitted"] != ref[:len(s["emitted"])]]
    out = {"source": "decode_qwen3_1p7b.json", "n_seq": N_SEQ, "steps": STEPS, "drafts": DRAFTS,
           "sequences": seqs, "left_greedy": diverged}
    (HERE / "verify_qwen3_1p7b.json").write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote verify_qwen3_1p7b.json; sequences leaving the plain greedy tokens: {diverged}")


if __name__ == "__main__":
    main()
