"""GPU: the exact_match surface's query-filtered functions (kgram_counts, kgram_query_counts, kgram_stats) and the
count mixture's features against the oracle (id-independent views: per valid position its context's totals, distinct
count and ranked next tokens; hit bitmaps; cnt with the cnt_top rule; the stats)."""

import numpy as np
import pytest
import torch

import oracle as O
from ngram_amd import data
from ngram_amd import exact_match as E

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def corpus():
    return data.make_corpus("c1", train_tokens=400_000, query_tokens=30_001, shard_tokens=150_000)


@pytest.fixture(scope="module")
def paths(corpus, tmp_path_factory):
    p, _ = corpus.write(tmp_path_factory.mktemp("em"))
    return p


def _bits(hits_bytes):
    pad = np.zeros((len(hits_bytes) + 63) // 64 * 64, np.uint8)
    pad[: len(hits_bytes)] = hits_bytes
    return np.packbits(pad, bitorder="little").view(np.uint64)


@pytest.mark.parametrize("k,top", [(1, 5), (2, 3), (3, 16), (6, 2)])
def test_kgram_counts(corpus, paths, k, top):
    q = corpus.query
    key_of, totals, distinct, offsets, nxt, ncnt, hits = E.kgram_counts(paths, q, k, top, 1 << 30)
    x, tgt = q[:-1], q[1:]
    o = O.query_counts(corpus.train, corpus.bounds, x, tgt, O.segments(x), k, ntop=top, hits=True)
    valid = key_of != np.uint32(0xFFFFFFFF)
    assert np.array_equal(valid, O.segments(x) >= k)
    ids = key_of[valid].astype(np.int64)
    assert np.array_equal(totals[ids], o["tot"][valid].astype(np.uint64))
    assert np.array_equal(np.minimum(distinct[ids], 65535), o["dist"][valid].astype(np.uint32))
    assert len(offsets) == len(totals) + 1 and offsets[-1] == len(nxt) == len(ncnt)
    for i in np.flatnonzero(valid)[:: max(1, int(valid.sum()) // 3000)]:
        c = int(key_of[i])
        a, b = int(offsets[c]), int(offsets[c + 1])
        m = min(top, int(o["dist"][i]))
        assert b - a == m
        assert np.array_equal(nxt[a:b], o["top_tok"][i, :m]) and np.array_equal(ncnt[a:b], o["top_cnt"][i, :m])
    assert np.array_equal(hits, _bits(o["hits"]))
    # train_tokens: the corpus' first tokens only
    r = E.kgram_counts(paths, q, k, top, 1 << 30, train_tokens=200_000)
    o2 = O.query_counts(corpus.train[:200_000], np.array([0, 150_000, 200_000]), x, tgt, O.segments(x), k, ntop=top)
    v2 = r[0] != np.uint32(0xFFFFFFFF)
    assert np.array_equal(r[1][r[0][v2].astype(np.int64)], o2["tot"][v2].astype(np.uint64))


def test_kgram_query_counts_breaks_and_cnt_top(corpus, paths):
    q = corpus.query
    breaks = [7000, 19000]
    r = E.kgram_query_counts(paths, q, 2, 4, 3, 1 << 30, breaks)
    x, tgt = q[:-1], q[1:]
    avail = O.segments(x, breaks)
    o = O.query_counts(corpus.train, corpus.bounds, x, tgt, avail, 2, cnt_top=3, ntop=4)
    assert np.array_equal(r[0] != np.uint32(0xFFFFFFFF), avail >= 2)
    assert np.array_equal(r[7], o["cnt"])
    assert (o["cnt"] != O.query_counts(corpus.train, corpus.bounds, x, tgt, avail, 2, cnt_top=1 << 30)["cnt"]).any()
    with pytest.raises(ValueError):
        E.kgram_query_counts(paths, q, 2, 4, 0, 1 << 30)
    with pytest.raises(ValueError):
        E.kgram_query_counts(paths, q, 2, 4, 3, 1 << 30, [len(q) - 1])


@pytest.mark.parametrize("k,depth", [(2, 4), (4, 8)])
def test_kgram_stats(corpus, paths, k, depth):
    q = corpus.query
    eligible, matched, ranks, hits = E.kgram_stats(paths, q, k, depth, 1 << 30)
    x, tgt = q[:-1], q[1:]
    av = O.segments(x)
    o = O.query_counts(corpus.train, corpus.bounds, x, tgt, av, k, ntop=depth)
    assert eligible == int((av >= k).sum()) and matched == int((o["tot"] > 0).sum())
    want = np.zeros(depth, np.uint64)
    for i in np.flatnonzero(o["tot"] > 0):
        hit = np.flatnonzero((o["top_tok"][i] == tgt[i]) & (o["top_cnt"][i] > 0))
        if len(hit):
            want[hit[0]] += 1
    assert np.array_equal(ranks, want)


def test_errors(paths, corpus):
    with pytest.raises(ValueError):
        E.kgram_counts([], corpus.query, 2, 4, 1)
    with pytest.raises(ValueError):
        E.kgram_counts(paths, corpus.query, 0, 4, 1)
    with pytest.raises(ValueError):
        E.kgram_counts(paths, corpus.query, 2, 4, 1, filter=np.zeros(3, np.uint64))
    with pytest.raises(AttributeError):
        E.val_scan
    assert E.CELLS == 168 and E.HEADER_BYTES == 1024


def test_features():
    rng = np.random.default_rng(5)
    L, n = 3, 50_000
    tot = rng.integers(0, 2 ** 32, size=(L, n), dtype=np.uint64)
    special = [0, 1, 2, 3, 4, 7, 8, 2 ** 24 - 1, 2 ** 24, 2 ** 24 + 1, 2 ** 31, 2 ** 32 - 1]
    tot[0, : len(special) * 16] = np.array(special * 16, np.uint64)
    tot[1] = rng.integers(0, 40, size=n)
    counts = np.zeros((3, L, n), np.int32)
    counts[0] = tot.astype(np.uint32).view(np.int32)
    counts[1] = rng.integers(0, 5, size=(L, n))
    counts[2] = (tot // rng.integers(1, 4, size=(L, n)).astype(np.uint64)).astype(np.uint32).view(np.int32)
    got = E.features(torch.from_numpy(counts).cuda())
    want = O.features(counts)
    for g, w, name in zip(got, want, ("tot", "dist", "cnt", "bin", "sparse")):
        assert np.array_equal(g.cpu().numpy(), w), name


@pytest.mark.parametrize("slots", [1, 3])
def test_train_hints_and_counts_match_brute_force(tmp_path, slots):
    """train_hints / train_counts (the rule "segment" over the shards in order) against the rules' brute force, on
    three small shard files with BOS tokens."""
    from ngram_amd import exact_match as X

    rng = np.random.default_rng(90 + slots)
    shards = []
    for j, n in enumerate((90, 120, 70)):
        t = rng.integers(0, 4, size=n).astype(np.uint16)
        t[rng.random(n) < 0.07] = O.BOS
        shards.append(t)
    files = []
    for j, t in enumerate(shards):
        f = tmp_path / f"s{j}.bin"
        data.write_shard(f, t)
        files.append(str(f))
    tok = np.concatenate(shards)
    bounds = [0, 90, 210, 280]
    levels, buckets = [1, 2, 3], [1, 2, 3, 4]
    got = X.train_hints(files, levels, 3, buckets, slots)
    want = O.brute_train_hints(tok, bounds, levels, buckets, 3, slots)
    if slots == 1:
        want = (want[0][:, 0], want[1][:, 0], want[2][:, 0], want[3][:, 0])
    for g, x, name in zip(got, want, ("cell", "tokens", "weights", "level")):
        assert g.shape == x.shape and np.array_equal(g, x), name
    assert (got[3] >= 0).sum() > 20
    tot, dist, cnt = X.train_counts(files, [3, 1])
    bw = O.brute_segment(tok, bounds, [], [1], 1, [3, 1])
    assert np.array_equal(tot, bw[3]) and np.array_equal(dist, bw[4]) and np.array_equal(cnt, bw[5])
    with pytest.raises(ValueError):
        X.train_hints(files, [2, 7], 3, buckets)
    with pytest.raises(ValueError):
        X.train_counts(files, [2, 2])
