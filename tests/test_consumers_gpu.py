"""GPU: the rows this build writes drop into the model-side consumers of the reference's hint runtime.

A hint directory is made from this build's own outputs:
  * validation rows and counts from the validation statistics (gpu_val_stats.build_stats);
  * causal training rows in one or two slots and their counts from train_hints / train_counts (the segment rule).
It is read back through the reader (`Hints`, HINT_NGRAM=1 for the count rows). Each batch then goes through what the
consumers compute from it (old_records/hint_runtime.py HintEmbedding :381-418, NgramMix :271-321 are the contract;
the checks below are written from that contract, not from its code):
  * a candidate mean: the embedding rows of a position's candidate tokens weighted by its row's weights, summed over
    the slots, zero where the row has no cell;
  * the probability of the target under a row: the weights of the candidates equal to the target;
  * interpolated Witten-Bell (Witten & Bell 1991; the interpolated form of Chen & Goodman 1998): per matched level j,
    lambda_j = tot_j / (tot_j + dist_j), P_j = lambda_j * cnt_j / tot_j + (1 - lambda_j) * P_{j-1}, from a unigram
    base P_0, levels in increasing length; an unmatched level passes P_{j-1} on;
  * a gate index from the deepest matched level: that level, the bin of its total among COUNT_EDGES, and whether it
    has one distinct continuation.
The test checks the invariants those consumers rely on: dtypes and shapes; cells below the table's; tokens below the
vocabulary; each row's weights a distribution (sum 1, up to u16 rounding) where it has a cell and all 0 where not;
cnt <= tot, dist <= tot, and dist >= 1 exactly where tot > 0, which makes every Witten-Bell level a proper
distribution (so every P_j lies in (0, 1]); the gate indices within their tables. It also checks that the losses
are finite."""

import numpy as np
import pytest
import torch

import oracle as O
from ngram_amd import data
from ngram_amd import exact_match as X
from ngram_amd import gpu_val_stats as G
from ngram_amd import hints as H

pytestmark = pytest.mark.gpu

COUNT_EDGES = (2, 3, 5, 9, 17, 33, 100, 1000, 10000)  # NgramMix.COUNT_EDGES (hint_runtime.py:271)


def _embed(rows, weight):
    """The candidate mean: per position and slot the weighted sum of its candidates' embedding rows, masked where the
    slot has no cell, then summed over the slots."""
    lead = rows.cell.shape
    tok = rows.tokens.reshape(-1, rows.tokens.shape[-1])
    w = rows.weights.reshape(-1, rows.weights.shape[-1])
    per = (weight[tok] * w[..., None]).sum(1) * (rows.cell.reshape(-1) > 0)[:, None].float()
    return per.reshape(*lead, -1).sum(1) if len(lead) == 2 else per


def _candidate_q(rows, targets):
    """Per position and slot, the row's probability of the target: the sum of the weights whose token is it."""
    tokens, weights = rows.tokens, rows.weights
    t = targets.view(-1, *([1] * (tokens.dim() - 1)))
    return torch.where(tokens == t, weights, torch.zeros_like(weights)).sum(-1)


def _witten_bell_log_q(targets, counts, unigram):
    """log P of the target under interpolated Witten-Bell over the count rows (levels in increasing length), in
    float64: lambda = tot / (tot + dist) per matched level, P = lambda * cnt / tot + (1 - lambda) * P_lower."""
    c = counts.double()
    tot, dist, cnt = c[:, 0], c[:, 1], c[:, 2]
    base = unigram.double() / unigram.double().sum()
    p = base[targets]
    for j in range(tot.shape[1]):
        t, d, n = tot[:, j], dist[:, j], cnt[:, j]
        m = t > 0
        lam = torch.where(m, t / (t + d).clamp_min(1), torch.zeros_like(t))
        assert torch.all((lam >= 0) & (lam < 1))
        ml = torch.where(m, n / t.clamp_min(1), torch.zeros_like(t))
        p = lam * ml + (1 - lam) * p
    return torch.log(p)


def _gate_index(counts):
    """(gate, sparse) indices of the deepest matched level (0: none matched): level d = 1..L of it, the bin of its
    total (how many COUNT_EDGES lie below it), and whether it has exactly one distinct continuation."""
    tot, dist = counts[:, 0].cpu().numpy(), counts[:, 1].cpu().numpy()
    n, L = tot.shape
    edges = np.asarray(COUNT_EDGES, np.float64)
    gate, sparse = np.zeros(n, np.int64), np.zeros(n, np.int64)
    for i in range(n):
        matched = np.flatnonzero(tot[i] > 0)
        if len(matched) == 0:
            continue
        j = matched[-1]
        d = j + 1
        gate[i] = d * (len(COUNT_EDGES) + 1) + int(np.searchsorted(edges, tot[i, j], side="left"))
        sparse[i] = d * 2 + int(dist[i, j] == 1)
    return gate, sparse


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
        lq = _witten_bell_log_q(targets, rows.counts, unigram)
        assert torch.isfinite(lq).all() and torch.all(lq <= 1e-9)
        gate, sparse = _gate_index(rows.counts[:2000])
        assert gate.max() < (len(count_levels) + 1) * (len(COUNT_EDGES) + 1) and gate.min() >= 0
        assert sparse.max() < 2 * (len(count_levels) + 1) and sparse.min() >= 0
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
