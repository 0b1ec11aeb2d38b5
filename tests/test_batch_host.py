"""Host logic of the batched decoder (pilm_amd.qwen3.Qwen3Batch): greedy draft
acceptance (src/engine.py:467-545) and the packing of several sequences'
block-aligned prompt chunks into batches.  No GPU: the model call is replaced
by a recorder."""
from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")

from pilm_amd import qwen3 as Q  # noqa: E402


def _rows(ids, vocab=8):
    x = torch.zeros((len(ids), vocab), dtype=torch.bfloat16)
    for r, i in enumerate(ids):
        x[r, i] = 1.0
    return x


@pytest.mark.parametrize("ids,drafts,want", [
    ([3, 4, 5, 6, 7], [3, 4, 5, 6], ([3, 4, 5, 6], 7)),      # all accepted: bonus token of the last row
    ([3, 4, 5, 6, 7], [3, 1, 5, 6], ([3], 4)),               # rejected at the second: that row's argmax
    ([3, 4, 5, 6, 7], [0, 4, 5, 6], ([], 3)),                # rejected at once
    ([2], [], ([], 2)),                                      # no drafts: a plain decode row
])
def test_accept_drafts(ids, drafts, want):
    assert Q.accept_drafts(_rows(ids), drafts) == want


def test_accept_drafts_first_index_of_ties():
    x = torch.zeros((2, 8), dtype=torch.bfloat16)
    x[0, 2] = x[0, 5] = 1.0          # argmax picks 2
    x[1, 1] = 1.0
    assert Q.accept_drafts(x, [5]) == ([], 2)
    assert Q.accept_drafts(x, [2]) == ([2], 1)


class _Recorder:
    def __init__(self, b):
        self.b, self.calls = b, []

    def __call__(self, groups, with_logits):
        rows = sum(len(t) for _, t in groups)
        assert rows <= self.b.max_rows
        for s, toks in groups:
            pos0 = self.b.cache_len[s]
            bs = self.b.cfg.block_size
            assert pos0 // bs == (pos0 + len(toks) - 1) // bs, "a chunk crosses a KV block"
        self.calls.append(([(s, len(t), self.b.cache_len[s]) for s, t in groups], with_logits))
        self.b.logits_rows.zero_()
        r = 0
        for s, toks in groups:
            r += len(toks)
            self.b.logits_rows[r - 1, s] = 1.0     # the last row of each group predicts its sequence id
        return rows


def _batch(max_rows, n_seqs):
    b = object.__new__(Q.Qwen3Batch)
    b.cfg = Q.Qwen3Config(block_size=16)
    b.max_rows = max_rows
    b.cache_len = [0] * n_seqs
    b.logits_rows = torch.zeros((max_rows, 32), dtype=torch.bfloat16)
    b._run = _Recorder(b)
    return b


def test_prefill_seqs_packs_block_aligned_chunks():
    lens = [40, 7, 16, 33, 1]
    b = _batch(40, len(lens))
    first = b.prefill_seqs(list(range(len(lens))), [[1] * n for n in lens])
    assert first == list(range(len(lens)))
    assert b.cache_len == lens
    done = {s: 0 for s in range(len(lens))}
    for groups, _ in b._run.calls:
        for s, n, pos0 in groups:
            assert pos0 == done[s]
            done[s] += n
    assert done == dict(enumerate(lens))
    assert max(sum(n for _, n, _ in g) for g, _ in b._run.calls) <= 40


def test_prefill_seqs_rejects_buffers_below_a_chunk():
    b = _batch(8, 1)
    with pytest.raises(ValueError, match="exceeds the batch buffers"):
        b.prefill_seqs([0], [[1] * 20])
