"""GPU: CountTable (exact_match's CountTable surface on libngram_amd.so) bit-exact against the oracle's restatement
of count_table.rs on seeded synthetic streams: query_counts with the CNT_TOP rule and without it, query_topk,
query_rows, sizes, and the errors of the reference's surface."""

import numpy as np
import pytest

import oracle as O
from ngram_amd import data
from ngram_amd.count_table import CountTable

pytestmark = pytest.mark.gpu

LEVELS = [1, 2, 3, 4, 6]


@pytest.fixture(scope="module")
def corpus():
    return data.make_corpus("c2", train_tokens=600_000, query_tokens=40_001, shard_tokens=250_000)


@pytest.fixture(scope="module")
def built(corpus, tmp_path_factory):
    d = tmp_path_factory.mktemp("shards")
    paths, _ = corpus.write(d)
    ct = CountTable.create(paths, LEVELS, 4, [])
    ct.build()
    return ct


@pytest.fixture(scope="module")
def reference(corpus):
    x, tgt = corpus.query[:-1], corpus.query[1:]
    avail = O.segments(x)
    ref = {}
    for k in LEVELS:
        ref[k] = O.table_counts(corpus.train, corpus.bounds, x, tgt, avail, k)
        ref[k]["cnt_all"] = O.table_counts(corpus.train, corpus.bounds, x, tgt, avail, k, cnt_top=1 << 30)["cnt"]
    return ref


def test_query_counts(built, corpus, reference):
    tot, dist, cnt = built.query_counts(corpus.query)
    assert tot.dtype == np.uint32 and dist.dtype == np.uint16 and cnt.dtype == np.uint32
    assert tot.shape == (len(corpus.query) - 1, len(LEVELS))
    for li, k in enumerate(LEVELS):
        o = reference[k]
        assert np.array_equal(tot[:, li], o["tot"]), k
        assert np.array_equal(dist[:, li], o["dist"]), k
        assert np.array_equal(cnt[:, li], o["cnt"]), k
    # the CNT_TOP rule matters at level 1 (the Zipf head has > 1024 distinct next tokens)
    assert (reference[1]["cnt"] != reference[1]["cnt_all"]).any()
    _, _, cnt_all = built.query_counts(corpus.query, top=1 << 16)
    for li, k in enumerate(LEVELS):
        assert np.array_equal(cnt_all[:, li], reference[k]["cnt_all"]), k


def test_query_topk(built, corpus, reference):
    tt, tc = built.query_topk(corpus.query, 4)
    for li, k in enumerate(LEVELS):
        assert np.array_equal(tt[:, li], reference[k]["top_tok"][:, :4]), k
        assert np.array_equal(tc[:, li], reference[k]["top_cnt"][:, :4]), k


@pytest.mark.parametrize("row_levels,entries", [([2, 4, 6], 8), ([1, 3], 5), ([6], 1)])
def test_query_rows(built, corpus, reference, row_levels, entries):
    buckets = [1, 2, 3, 4, 5, 6]
    got = built.query_rows(corpus.query, row_levels, buckets, entries)
    want = O.table_rows(reference, row_levels, buckets, entries)
    for g, w, name in zip(got, want, ("cell", "next", "weights", "level")):
        assert g.dtype == w.dtype, name
        assert np.array_equal(g, w), name


def test_sizes(built, reference):
    for (k, contexts, pairs, nbytes), kk in zip(built.sizes(), LEVELS):
        assert k == kk and contexts == reference[k]["contexts"] and pairs == reference[k]["pairs"] and nbytes > 0
    assert built.levels == LEVELS and built.tokens == 600_000


def test_errors(corpus, built):
    with pytest.raises(ValueError):
        CountTable.create(corpus.shards(), [3, 2], 1, [])
    with pytest.raises(ValueError):
        CountTable.create([], [2], 1, [])
    ct = CountTable.create(corpus.shards(), [2], 1, [])
    with pytest.raises(ValueError):
        ct.query_counts(corpus.query)  # not built
    with pytest.raises(ValueError):
        built.query_counts(corpus.query, top=2000)
    with pytest.raises(ValueError):
        built.query_counts(np.array([5], np.uint16))
    with pytest.raises(ValueError):
        built.query_rows(corpus.query, [5], [5])  # not a table level
    with pytest.raises(ValueError):
        built.query_rows(corpus.query, [2], [3])  # not in buckets
    ct.build()
    with pytest.raises(ValueError):
        ct.build()
    ct.release()
    with pytest.raises(ValueError):
        ct.query_counts(corpus.query)


def test_overflow_reruns(corpus, reference, monkeypatch):
    import ngram_amd.count_table as T

    monkeypatch.setattr(T, "LOAD", 1e9)  # 65536-slot tables: level 4 overflows them and reruns bigger
    ct = CountTable.create(corpus.shards(), [4], 1, [])
    ct.build()
    assert ct.reruns[4] > 0
    tot, dist, cnt = ct.query_counts(corpus.query)
    assert np.array_equal(tot[:, 0], reference[4]["tot"]) and np.array_equal(cnt[:, 0], reference[4]["cnt"])


def test_escaped_counts(corpus, reference, monkeypatch):
    """Packed words with a 4-bit count field (context bits forced to 44): every count of 15 or more lives in the
    escape table, for the records' totals and tops and the CNT_TOP thresholds (the queries' counts come from the
    slabs, which hold them whole)."""
    from ngram_amd import partcount as P

    monkeypatch.setattr(P, "PACK32_MIN_BITS", 44)
    ct = CountTable.create(corpus.shards(), [1, 3], 1, [])
    ct.build()
    assert all(lv.cb == 44 for lv in ct.tables)
    assert int((ct.tables[0].esc[0] != -1).sum().item()) > 100  # level 1 holds many counts >= 15
    tot, dist, cnt = ct.query_counts(corpus.query)
    _, _, cnt_all = ct.query_counts(corpus.query, top=1 << 16)
    tt, tc = ct.query_topk(corpus.query, 8)
    for li, k in enumerate([1, 3]):
        o = reference[k]
        assert np.array_equal(tot[:, li], o["tot"]) and np.array_equal(dist[:, li], o["dist"]), k
        assert np.array_equal(cnt[:, li], o["cnt"]) and np.array_equal(cnt_all[:, li], o["cnt_all"]), k
        assert np.array_equal(tt[:, li], o["top_tok"]) and np.array_equal(tc[:, li], o["top_cnt"]), k


def test_cache_ladder_rung(corpus, tmp_path):
    from ngram_amd.cache_ladder import GpuCountIndex

    paths, _ = corpus.write(tmp_path)
    idx = GpuCountIndex.create(paths, 500_000, 4, [])
    stats = idx.build()
    train = corpus.train[:500_000]
    bounds = np.array([0, 250_000, 500_000])
    x = corpus.query[:-1]
    from numpy.lib.stride_tricks import sliding_window_view

    for k in (6, 10, 20):
        # every (k + 1)-window within a shard is an occurrence: distinct windows = pairs, distinct k-prefixes = contexts
        wins = np.concatenate([sliding_window_view(train[a:b], k + 1) for a, b in zip(bounds[:-1], bounds[1:])])
        pairs = np.unique(wins, axis=0)
        contexts = np.unique(pairs[:, :k], axis=0)
        assert stats[f"contexts_{k}"] == len(contexts) and stats[f"pairs_{k}"] == len(pairs), k
    assert stats["tokens"] == 500_000 and stats["seconds"] > 0
    with pytest.raises(ValueError):
        GpuCountIndex.create(paths, 10_000_000)
