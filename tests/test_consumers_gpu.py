"""GPU: the rows this build writes drop into the model-side consumers of the reference's hint runtime.

A hint directory is made from this build's own outputs:
  * validation rows and counts from the validation statistics (gpu_val_stats.build_stats);
  * causal training rows in one or two slots and their counts from train_hints / train_counts (the segment rule).
It is read back through the reader (`Hints`, HINT_NGRAM=1 for the count rows). Each batch then goes through the
consumers' forward arithmetic, restated here from old_records/hint_runtime.py (the reference's module needs
Python >= 3.12 and its experiment framework, so it is read, not imported):
  * HintEmbedding.forward (:381-396): embedding_bag of the candidates with per-sample weights, the slots summed;
  * HintEmbedding.mixed_nll's candidate probabilities (:398-418);
  * NgramMix.gates and log_q (:289-321).
The test checks the invariants those consumers rely on: dtypes and shapes; cells below the table's; tokens below the
vocabulary; each row's weights a distribution (sum 1, up to u16 rounding) where it has a cell and all 0 where not;
cnt <= tot, dist <= tot, and dist >= 1 exactly where tot > 0, which makes every Witten-Bell level a proper
distribution. It also checks that the losses are finite."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from ngram_amd import data
from ngram_amd import exact_match as X
from ngram_amd import gpu_val_stats as G
from ngram_amd import hints as H

pytestmark = pytest.mark.gpu

COUNT_EDGES = (2, 3, 5, 9, 17, 33, 100, 1000, 10000)  # NgramMix.COUNT_EDGES (hint_runtime.py:271)


def _embed(rows, weight):
    """HintEmbedding.forward's candidate mean (hint_runtime.py:388-395), without the learned scales."""
    cell, tokens, weights = rows.cell, rows.tokens, rows.weights
    if cell.dim() == 2:
        cell, tokens, weights = cell.flatten(), tokens.flatten(0, 1), weights.flatten(0, 1)
    mean = F.embedding_bag(tokens, weight, per_sample_weights=weights, mode="sum")
    hint = mean * (cell > 0)[:, None]
    if rows.cell.dim() == 2:
        hint = hint.view(*rows.cell.shape, -1).sum(1)
    return hint


def _candidate_q(rows, targets):
    """mixed_nll's per-slot probability of the target (hint_runtime.py:410-412)."""
    cell, tokens, weights = rows.cell, rows.tokens, rows.weights
    if cell.dim() == 1:
        cell, tokens, weights = cell[:, None], tokens[:, None], weights[:, None]
    return (weights * (tokens == targets[:, None, None])).sum(-1)


def _ngram_log_q(targets, counts, unigram, levels):
    """NgramMix.log_q with its initial parameters (gamma 0: g_j = 1; hint_runtime.py:305-320)."""
    tot, dist, cnt = counts.float().unbind(1)
    assert tot.shape[1] == levels
    p = torch.log_softmax(torch.log(unigram.clamp_min(1e-12)), 0)[targets].exp()
    for j in range(levels):
        matched = tot[:, j] > 0
        gd = dist[:, j]
        den = torch.where(matched, tot[:, j] + gd, torch.ones_like(gd))
        p = torch.where(matched, (cnt[:, j] + gd * p) / den, p)
    return torch.log(p.clamp_min(1e-30))


def _gates(counts, levels):
    """NgramMix.gates (hint_runtime.py:289-303): the deepest matched level's gate and sparse index."""
    tot, dist = counts[:, 0].float(), counts[:, 1].float()
    matched = tot > 0
    level = torch.arange(1, levels + 1, device=tot.device)
    deepest = (matched.long() * level).amax(1) - 1
    at = deepest.clamp_min(0)[:, None]
    bins = sum((tot > e).long() for e in COUNT_EDGES)
    dbin = torch.gather(bins, 1, at)[:, 0]
    sparse = (torch.gather(dist, 1, at)[:, 0] == 1).long()
    d = deepest + 1
    hit = deepest >= 0
    return torch.where(hit, d * (len(COUNT_EDGES) + 1) + dbin, 0), torch.where(hit, d * 2 + sparse, 0)


def _check_rows(rows, n, slots, cells, count_levels):
    lead = (n,) if slots == 1 else (n, slots)
    assert rows.cell.shape == lead and rows.cell.dtype == torch.int64
    assert rows.tokens.shape == (*lead, H.ENTRIES) and rows.tokens.dtype == torch.int64
    assert rows.weights.shape == (*lead, H.ENTRIES) and rows.weights.dtype == torch.float32
    assert int(rows.cell.min()) >= 0 and int(rows.cell.max()) < cells
    assert int(rows.tokens.min()) >= 0 and int(rows.tokens.max()) < H.VOCAB
    s = rows.weights.sum(-1)
    has = rows.cell > 0
    assert torch.all((s[has] - 1).abs() < H.ENTRIES / H.WEIGHT_ONE) and torch.all(s[~has] == 0)
    c = rows.counts
    assert c.shape == (n, 3, len(count_levels)) and c.dtype == torch.float32
    tot, dist, cnt = c.unbind(1)
    assert torch.all(cnt <= tot) and torch.all(dist <= tot) and torch.all((dist >= 1) == (tot > 0))
    return has


@pytest.mark.parametrize("slots", [1, 2])
def test_rows_drop_into_the_consumers(tmp_path, monkeypatch, slots):
    corpus = data.make_corpus("c3", train_tokens=600_000, query_tokens=40_001, shard_tokens=200_000)
    shards = corpus.shards()
    files = []
    for j, s in enumerate(shards):
        f = tmp_path / f"train_{j:04d}.bin"
        data.write_shard(f, s)
        files.append(str(f))
    levels, count_levels = (6, 10, 20), G.ALL_LEVELS
    # training rows and counts: causal (the segment rule) over the shards in order
    cell, tokens, weights, level = X.train_hints(files, levels, H.ENTRIES, H.BUCKETS, slots)
    tot, dist, cnt = X.train_counts(files, count_levels)
    bounds = np.cumsum([0] + [len(s) for s in shards])
    train = [(cell[a:b], tokens[a:b], weights[a:b]) for a, b in zip(bounds[:-1], bounds[1:])]
    train_counts = [(tot[a:b], dist[a:b], cnt[a:b]) for a, b in zip(bounds[:-1], bounds[1:])]
    # validation rows and counts: the validation statistics over every shard
    tok, sizes, starts, _ = data.device_tokens(shards)
    x, tgt, avail = G.val_queries(corpus.query)
    res = G.build_stats(tok, sizes, starts, x, tgt, avail, levels=count_levels, variants=(levels,))
    host = G.host_outputs(res)
    n = len(host["cell"][0])
    val = (host["cell"][0], host["tokens"][0], host["weights"][0])
    if slots > 1:  # one slot of deepest rows, the others empty (the layout the reader serves)
        val = tuple(np.concatenate([a[:, None], np.zeros_like(a[:, None]).repeat(slots - 1, 1)], 1) for a in val)
    d = H.write_hint_dir(tmp_path / "hints", levels, val, train, val_counts=(host["tot"], host["dist"], host["cnt"]),
                         train_counts=train_counts, unigram_base=H.unigram(shards[0]), count_levels=count_levels,
                         slots=slots, val_tokens=n)
    monkeypatch.setenv("HINT_NGRAM", "1")
    hints = H.Hints(d)
    weight = torch.randn(H.VOCAB, 64, device="cuda")
    unigram = torch.from_numpy(hints.unigram).cuda()
    assert unigram.shape == (H.VOCAB,) and abs(float(unigram.sum()) - 1) < 1e-3
    cells = H.cells(H.BUCKETS)
    batches = [(hints.val_span(0, n), corpus.query[1 : n + 1])]
    for j, s in enumerate(shards):
        m = len(s) - 1
        batches.append((hints.train_span(j, 0, m), s[1 : m + 1]))
    hinted = 0
    for rows, nxt in batches:
        m = rows.cell.shape[0]
        has = _check_rows(rows, m, slots, cells, count_levels)
        hinted += int(has.any(-1).sum() if slots > 1 else has.sum())
        targets = torch.from_numpy(nxt.astype(np.int64)).cuda()
        hint = _embed(rows, weight)
        assert hint.shape == (m, 64) and torch.isfinite(hint).all()
        q = _candidate_q(rows, targets)
        assert torch.all((q >= 0) & (q <= 1 + 1e-6))
        lq = _ngram_log_q(targets, rows.counts, unigram, len(count_levels))
        assert torch.isfinite(lq).all() and torch.all(lq <= 1e-6)
        gate, sparse = _gates(rows.counts, len(count_levels))
        assert int(gate.max()) < (len(count_levels) + 1) * (len(COUNT_EDGES) + 1)
        assert int(sparse.max()) < 2 * (len(count_levels) + 1)
    assert hinted > 1000
    # the causal rows at this scale against the oracle's restatement (contexts of at most 8 tokens: levels 4 and 6)
    # over the first shard, whose positions see only that shard's occurrences
    seg = np.zeros(len(shards[0]), bool)
    seg[0] = True
    seg |= shards[0] == O.BOS
    si = (np.cumsum(seg) - 1).astype(np.uint32)
    want = O.online(shards[0], [0, len(shards[0])], si, si, [4, 6], list(H.BUCKETS), H.ENTRIES, [], 0, int(si[-1]) + 1)
    got = X.train_hints(files[:1], [4, 6], H.ENTRIES, H.BUCKETS, slots)
    for g, w in zip(got[:3], want[:3]):
        assert np.array_equal(g if slots == 1 else g[:, 0], w)
    assert (want[0] != 0).sum() > 1000
