"""GPU: ragged and degenerate inputs through every counting path, bit-exact against the oracle: an empty shard, shards
shorter than the contexts, a shard of BOS tokens only, token ids at the top of the vocabulary, a query stream whose
segments are mostly shorter than the levels, contexts longer than any shard, and query positions that match nothing."""

import numpy as np
import pytest
import torch

import oracle as O
from ngram_amd import counts as C
from ngram_amd import data
from ngram_amd import gpu_val_stats as G
from ngram_amd.lib import Lib
from ngram_amd.count_table import CountTable
from ngram_amd.longest import _segments, longest_match

pytestmark = pytest.mark.gpu

BOS = 50256


@pytest.fixture(scope="module")
def ragged():
    rng = np.random.default_rng(7)
    small = rng.integers(0, 40, 30_000).astype(np.uint16)  # 40 token ids: long repeated contexts
    small[rng.random(30_000) < 0.01] = BOS
    top = rng.choice(np.array([50250, 50251, 50255, BOS], np.uint16), 5_000)  # ids at the vocabulary's top
    period = np.tile(np.arange(100, 117, dtype=np.uint16), 300)  # a periodic shard: matches longer than 64
    shards = [np.array([5, 6, 7], np.uint16), np.zeros(0, np.uint16), np.array([9], np.uint16),
              np.full(50, BOS, np.uint16), small, np.array([1, 2, 3, 4, 5, 6, 7], np.uint16), top, period]
    # queries: copies of corpus spans, a BOS-dense stretch (segments of 1-3 tokens), tokens never seen in the corpus
    q = np.concatenate([small[100:2100], period[:500], np.tile(np.array([BOS, 3, BOS, 4, 5], np.uint16), 200),
                        np.full(300, 30_000, np.uint16), top[:1000], rng.integers(0, 40, 3000).astype(np.uint16)])
    bounds = np.cumsum([0] + [len(s) for s in shards])
    return shards, np.concatenate(shards), bounds, q


@pytest.mark.parametrize("mode", ["dense", "list"])
def test_counts_on_ragged_shards(ragged, mode):
    shards, train, bounds, q = ragged
    levels = (1, 2, 3, 5, 8, 20)
    cb = C.CountBuild(shards, levels=levels, level_shards={}, topk=4)
    if mode == "list":  # every gated level probes the previous level's hits listed in memory
        cb.engine.density = {k: 0.0 for k in levels}
    cb.start_load(1)
    x, tgt, avail = C.queries(q, [], "cuda")
    out = cb.counts(x, tgt, avail, stats=True).cpu().numpy()
    xs, ts = q[:-1], q[1:]
    av = O.segments(xs)
    for li, k in enumerate(levels):
        o = O.query_counts(train, bounds, xs, ts, av, k, cnt_top=1 << 30, ntop=4)
        assert np.array_equal(out[0, li].view(np.uint32), o["tot"]), (mode, k)
        assert np.array_equal(out[1, li].astype(np.uint16), o["dist"]), (mode, k)
        assert np.array_equal(out[2, li].view(np.uint32), o["cnt"]), (mode, k)
        assert np.array_equal(cb.top_tok[li].cpu().numpy().view(np.uint16), o["top_tok"][:, :4]), (mode, k)
        assert np.array_equal(cb.top_cnt[li].cpu().numpy().view(np.uint32), o["top_cnt"][:, :4]), (mode, k)
    assert (out[0, levels.index(20)] > 0).any()  # the periodic shard matches at 20


def test_val_stats_on_ragged_shards(ragged):
    shards, train, bounds, q = ragged
    tok, sizes, starts, L = data.device_tokens(shards)
    x, tgt, avail = G.val_queries(q)
    res = G.build_stats(tok, sizes, starts, x, tgt, avail)
    counts = res["counts"].cpu().numpy()
    xs, ts = q[:-1], q[1:]
    av = O.segments(xs)
    for li, k in enumerate(G.ALL_LEVELS):
        o = O.query_counts(train, bounds, xs, ts, av, k)
        assert np.array_equal(counts[0, li].view(np.uint32), o["tot"]), k
        assert np.array_equal(counts[2, li].view(np.uint32), o["cnt"]), k


@pytest.mark.parametrize("cap", [64, 3])
def test_longest_on_ragged_shards(ragged, cap):
    shards, train, bounds, q = ragged
    tok, sizes, starts, L = data.device_tokens(shards)
    xs = q[:-1]
    xt = torch.from_numpy(xs.view(np.int16).copy()).cuda()
    av = _segments(xt, Lib())
    length, nxt, cnt, _ = longest_match(tok, xt, av, cap)
    want = O.longest_match(train, bounds, xs, O.segments(xs), cap)
    assert np.array_equal(length.cpu().numpy().view(np.uint32), want[0])
    assert np.array_equal(nxt.cpu().numpy().view(np.uint16), want[1])
    assert np.array_equal(cnt.cpu().numpy().view(np.uint32), want[2])
    assert want[0].max() == cap and (want[0] == 0).any()


def test_count_table_on_ragged_shards(ragged):
    shards, train, bounds, q = ragged
    levels = [1, 2, 4, 8]
    ct = CountTable.create(shards, levels, 1, [])
    ct.build()
    tot, dist, cnt = ct.query_counts(q)
    tt, tc = ct.query_topk(q, 8)
    xs, ts = q[:-1], q[1:]
    av = O.segments(xs)
    for li, k in enumerate(levels):
        o = O.table_counts(train, bounds, xs, ts, av, k)
        assert np.array_equal(tot[:, li], o["tot"]) and np.array_equal(dist[:, li], o["dist"]), k
        assert np.array_equal(cnt[:, li], o["cnt"]), k
        assert np.array_equal(tt[:, li], o["top_tok"]) and np.array_equal(tc[:, li], o["top_cnt"]), k
