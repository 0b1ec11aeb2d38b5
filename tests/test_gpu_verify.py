"""GPU: speculative (MTP) verify under continuous batching, against the oracle.

The reference verifies one sequence's last token and its drafts as one
model call over 1 + k rows, lm_head over every row, and accepts the drafts
while each equals the argmax of the row before it (src/engine.py:416-545).
Under continuous batching (src/runtime/scheduler/scheduler.py:70-178) the
device takes every running sequence's rows as one M: 16 sequences x
(1 + 4 drafts) is an M = 80 call per linear, attention per sequence on its
own block table in a shared KV pool.

Checked here:
  * the two-layer model, W4A16 g128 and int8 per-row weights: every verify
    row's bf16 logits bit-identical to the oracle's per-sequence model call
    (oracle/decoder.py), the accepted drafts
    and next token per sequence equal to the oracle's, and the emitted tokens
    equal to plain greedy decoding (what greedy speculation must give);
  * Qwen3-1.7B W4A16 g128: 16 sequences on the 128-token prompt of the
    reference's fixture, speculating with drafts taken from the reference's
    own greedy tokens and corrupted at varying positions; every verify row's
    logits, accepted drafts and next token equal to the oracle's (a fixture:
    the oracle needs minutes per sequence at this size).  A verify row is not
    always bit-identical to the one-row decode step at its position (torch's
    P.V partial sums depend on the masked row length), so these tokens may
    leave the plain greedy ones at a near tie, in the reference too.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

from oracle import decoder as OD

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _bits(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _fixture(name):
    return json.loads((GOLDEN / f"decode_{name}.json").read_text())


def _corrupt(tok, vocab, salt):
    return (tok + 1 + salt) % vocab


def _drafts(greedy, start, n, bad, vocab, salt):
    """n drafts following greedy[start - 1]; draft `bad` (if < n) is wrong."""
    d = list(greedy[start:start + n])
    if bad < n:
        d[bad] = _corrupt(d[bad], vocab, salt)
        assert d[bad] != greedy[start + bad]
    return d


@pytest.mark.parametrize("weights", ["w4g128", "w8"])
def test_batched_verify_two_layer_matches_oracle(dev, weights):
    """W4A16 g128, and int8 per-row weights as the reference's W8A32
    quantization runs them in a bf16 model (W8A16, the Qwen3-8B MTP
    configuration's format), on the two-layer model."""
    from pilm_amd import qwen3 as Q
    from pilm_amd import synth_model as SM
    fx = _fixture("tiny")
    c = dict(fx["config"])
    c["weights"] = weights
    n_seq, n_greedy = 16, 12
    prompts = [SM.token_ids(200 + i, 3 + 7 * i, c["vocab"]) for i in range(n_seq)]
    c["prompt"], c["new_tokens"] = max(len(p) for p in prompts), n_greedy + 4
    V = c["vocab"]

    # Two verify steps per sequence.  Step 1: 4 drafts, the j-th wrong
    # (j = i % 5; 4 means all right).  Step 2: 0 .. 4 drafts, one maybe wrong.
    plan = []
    for i in range(n_seq):
        j1 = i % 5
        n2, j2 = i % 5, (3 * i + 1) % 5
        plan.append((j1, n2, j2))

    _say(f"[gpu] batched verify, two-layer {weights} model: oracle greedy and verify rows (CPU)")
    od = OD.OracleDecoder(c)
    greedy, want = [], []
    for i in range(n_seq):
        g = od.generate(prompts[i], n_greedy)
        greedy.append(g)
        j1, n2, j2 = plan[i]
        p = len(prompts[i])
        d1 = _drafts(g, 1, 4, j1, V, i)
        rows1 = od.forward([g[0]] + d1, p, all_rows=True)
        a1 = min(j1, 4)
        d2 = _drafts(g, 2 + a1, n2, j2, V, i + 7)
        rows2 = od.forward([g[1 + a1]] + d2, p + 1 + a1, all_rows=True)
        want.append(((d1, rows1), (d2, rows2)))

    _say("[gpu] batched verify, two-layer model: weights, prefill")
    w = Q.Qwen3Weights.synthetic(Q.Qwen3Config.from_dict(c), c["seed"], c["std"], device=dev)
    b = Q.Qwen3Batch(w, n_seqs=n_seq, max_positions=c["prompt"] + c["new_tokens"] + 1, max_rows=96)
    first = [b.prefill_seq(i, prompts[i]) for i in range(n_seq)]
    assert first == [g[0] for g in greedy]

    last = first
    for step in range(2):
        drafts = [want[i][step][0] for i in range(n_seq)]
        rows = sum(1 + len(d) for d in drafts)
        _say(f"[gpu] batched verify, two-layer model: step {step + 1}, M = {rows}")
        out = b.verify(last, drafts)
        r0 = 0
        for i in range(n_seq):
            d, ref_rows = want[i][step]
            got = _bits(b.logits_rows[r0:r0 + 1 + len(d)])
            assert np.array_equal(got, ref_rows), f"sequence {i} step {step + 1}: logits differ from the oracle"
            r0 += 1 + len(d)
            ids = [OD.argmax_bf16(r) for r in ref_rows]
            acc = []
            for k, t in enumerate(d):
                if ids[k] != t:
                    break
                acc.append(t)
            nxt = ids[len(acc)]
            assert out[i] == (acc, nxt), f"sequence {i} step {step + 1}"
            emitted = [last[i]] + acc + [nxt]
            pos = b.cache_len[i] - len(prompts[i])           # tokens of the sequence now in the cache
            assert emitted == greedy[i][pos - 1 - len(acc):pos + 1], f"sequence {i}: not the greedy tokens"
        last = [o[1] for o in out]


def test_batched_speculation_qwen3_1p7b_matches_oracle(dev):
    """Qwen3-1.7B W4A16 g128: 16 sequences on the reference fixture's prompt,
    8 verify steps of M = 80, all on the exact kernels.  Each step's drafts,
    accepted drafts, next token and the sha256 of the five verify rows' bf16
    logits must equal what the oracle computed for that sequence alone
    (tests/golden/verify_qwen3_1p7b.json, written by gen_verify_fixture.py)."""
    from pilm_amd import qwen3 as Q
    fx = _fixture("qwen3_1p7b")
    path = GOLDEN / "verify_qwen3_1p7b.json"
    if not path.exists():
        pytest.skip("tests/golden/verify_qwen3_1p7b.json not generated (gen_verify_fixture.py)")
    sv = json.loads(path.read_text())
    c = fx["config"]
    n_seq, steps = sv["n_seq"], sv["steps"]
    _say("[gpu] batched speculation Qwen3-1.7B: weights")
    w = Q.Qwen3Weights.synthetic(Q.Qwen3Config.from_dict(c), c["seed"], c["std"], device=dev)
    b = Q.Qwen3Batch(w, n_seqs=n_seq, max_positions=c["prompt"] + 5 * steps + 8, max_rows=96)
    _say(f"[gpu] batched speculation Qwen3-1.7B: prefill {n_seq} x {len(fx['prompt'])} tokens")
    first = b.prefill_seqs(list(range(n_seq)), [fx["prompt"]] * n_seq)
    assert first == [q["first"] for q in sv["sequences"]]
    last = first
    for step in range(steps):
        want = [q["steps"][step] for q in sv["sequences"]]
        _say(f"[gpu] batched speculation Qwen3-1.7B: verify step {step + 1}, M = {sum(1 + len(x['drafts']) for x in want)}")
        out = b.verify(last, [x["drafts"] for x in want])
        r0 = 0
        for i, x in enumerate(want):
            rows = 1 + len(x["drafts"])
            assert OD.sha_u16(_bits(b.logits_rows[r0:r0 + rows])) == x["rows_sha"], \
                f"sequence {i} step {step + 1}: verify logits differ from the oracle"
            assert out[i] == (x["accepted"], x["next"]), f"sequence {i} step {step + 1}"
            r0 += rows
        last = [o[1] for o in out]
    for i, q in enumerate(sv["sequences"]):
        assert b.cache_len[i] == len(fx["prompt"]) + len(q["emitted"]) - 1


def test_batched_verify_matrix_cores_close_to_exact(dev):
    """Qwen3Batch(exact=False): batches of 64 rows or more on the matrix cores.
    On the two-layer model, 16 sequences x 5 rows after their prompts: every
    verify row's logits within 5e-2 of the row's largest magnitude of the
    exact mode's (two layers of 1e-2 GEMM tolerance, prefill included), and
    the rows' argmax equal wherever the exact row's top two are apart by
    more than that."""
    from pilm_amd import qwen3 as Q
    from pilm_amd import synth_model as SM
    c = dict(_fixture("tiny")["config"])
    n_seq = 16
    prompts = [SM.token_ids(300 + i, 20 + 3 * i, c["vocab"]).tolist() for i in range(n_seq)]
    w = Q.Qwen3Weights.synthetic(Q.Qwen3Config.from_dict(c), c["seed"], c["std"], device=dev)
    rows = {}
    for exact in (True, False):
        _say(f"[gpu] batched verify, two-layer model, exact={exact}: prefill and one step, M = 80")
        b = Q.Qwen3Batch(w, n_seqs=n_seq, max_positions=max(len(p) for p in prompts) + 8, max_rows=96, exact=exact)
        b.prefill_seqs(list(range(n_seq)), prompts)
        b.verify([1 + i for i in range(n_seq)], [[7, 8, 9, 10]] * n_seq)
        rows[exact] = b.logits_rows[:80].to(torch.float32).cpu()
    a, m = rows[True], rows[False]
    scale = a.abs().amax(dim=1)
    err = ((a - m).abs().amax(dim=1) / scale).max().item()
    assert err <= 5e-2, f"matrix-core verify rows differ by {err:.3g} of the row's largest logit"
    top2 = a.topk(2, dim=1).values
    clear = (top2[:, 0] - top2[:, 1]) > 5e-2 * scale
    assert torch.equal(a.argmax(dim=1)[clear], m.argmax(dim=1)[clear])


def test_w8_8b_shapes_decode_and_verify_match_oracle(dev):
    """Two layers with Qwen3-8B's shapes (hidden 4096, 32 q / 8 kv heads,
    intermediate 12288; a 4096-token vocabulary keeps the oracle fast) and
    int8 per-row weights, the MTP configuration's format: the greedy tokens
    and every step's logits of one sequence, then one batched verify step of
    4 sequences x 5 rows, bit for bit against the oracle run per sequence."""
    from pilm_amd import qwen3 as Q
    from pilm_amd import synth_model as SM
    c = {"layers": 2, "hidden": 4096, "heads": 32, "kv_heads": 8, "head_dim": 128, "intermediate": 12288,
         "vocab": 4096, "eps": 1e-6, "rope_theta": 1e6, "partial_rotary": 1.0, "block_size": 16, "group_size": 128,
         "std": 0.02, "seed": 23, "weights": "w8", "prompt": 20, "new_tokens": 6}
    prompt = SM.token_ids(51, c["prompt"], c["vocab"]).tolist()
    _say("[gpu] 8B-shaped W8 model: oracle weights and greedy decode (CPU)")
    od = OD.OracleDecoder(c)
    want_sha = []
    want = od.generate(prompt, c["new_tokens"], on_logits=lambda i, lg: want_sha.append(OD.sha_u16(lg)))
    _say("[gpu] 8B-shaped W8 model: device weights and decode")
    w = Q.Qwen3Weights.synthetic(Q.Qwen3Config.from_dict(c), c["seed"], c["std"], device=dev, hashes=True)
    assert w.quantized_sha == od.qsha
    dec = Q.Qwen3Decoder(w, max_positions=c["prompt"] + c["new_tokens"] + 1, max_new_tokens=c["new_tokens"])
    shas = []
    toks = dec.generate(prompt, c["new_tokens"], on_logits=lambda i, lg: shas.append(OD.sha_u16(_bits(lg))))
    first = next((i for i, (a, b) in enumerate(zip(shas, want_sha)) if a != b), None)
    assert first is None, f"logits differ first at step {first}"
    assert toks == want

    n_seq = 4
    prompts = [SM.token_ids(60 + i, 5 + 3 * i, c["vocab"]).tolist() for i in range(n_seq)]
    drafts = [[(7 * i + j) % c["vocab"] for j in range(4)] for i in range(n_seq)]
    _say("[gpu] 8B-shaped W8 model: oracle verify rows per sequence (CPU)")
    want_rows, last = [], []
    for i in range(n_seq):          # the oracle's cache is rewritten from position 0 for each sequence
        g = od.generate(prompts[i], 1)
        last.append(g[0])
        want_rows.append(od.forward([g[0]] + drafts[i], len(prompts[i]), all_rows=True))
    _say("[gpu] 8B-shaped W8 model: batched prefill and one verify step, M = 20")
    b = Q.Qwen3Batch(w, n_seqs=n_seq, max_positions=max(len(p) for p in prompts) + 9, max_rows=32)
    assert b.prefill_seqs(list(range(n_seq)), prompts) == last
    b.verify(last, drafts)
    r0 = 0
    for i in range(n_seq):
        got = _bits(b.logits_rows[r0:r0 + 5])
        assert np.array_equal(got, want_rows[i]), f"sequence {i}: verify rows differ from the oracle"
        r0 += 5
