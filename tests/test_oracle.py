"""CPU: the oracle pinned against brute force, closed forms and hand-computed cases (no GPU)."""

import numpy as np
import pytest
import torch

import oracle as O
from ngram_amd import data


def _case(rng, vocab, n_shards, max_len, nq):
    shards = [rng.integers(0, vocab, size=int(rng.integers(0, max_len))).astype(np.uint16) for _ in range(n_shards)]
    for s in shards:
        s[rng.random(len(s)) < 0.08] = O.BOS
    train = np.concatenate(shards) if shards else np.zeros(0, np.uint16)
    bounds = np.cumsum([0] + [len(s) for s in shards]).astype(np.int64)
    q = rng.integers(0, vocab, size=nq).astype(np.uint16)
    q[rng.random(nq) < 0.08] = O.BOS
    return shards, train, bounds, q[:-1], q[1:]


@pytest.mark.parametrize("seed", range(12))
def test_restatements_match_brute_force(seed):
    rng = np.random.default_rng(seed)
    shards, train, bounds, x, tgt = _case(rng, int(rng.integers(2, 7)), int(rng.integers(1, 4)), 80, 50)
    avail = O.segments(x)
    for k in (1, 2, 3, 4, 5):
        b = O.brute_counts(shards, x, tgt, avail, k, cnt_top=2, ntop=3)
        a = O.query_counts(train, bounds, x, tgt, avail, k, cnt_top=2, ntop=3)
        c = O.table_counts(train, bounds, x, tgt, avail, k, cnt_top=2, ntop=3)
        for name in ("tot", "dist", "cnt", "top_tok", "top_cnt"):
            assert np.array_equal(a[name], b[name]), (k, name)
            assert np.array_equal(c[name], b[name]), (k, name, "table")


@pytest.mark.parametrize("seed", range(4))
def test_longest_match_matches_brute_force(seed):
    rng = np.random.default_rng(100 + seed)
    shards, train, bounds, x, tgt = _case(rng, 3, 2, 60, 40)
    avail = O.segments(x)
    got = O.longest_match(train, bounds, x, avail, 7)
    want = O.brute_longest(shards, x, avail, 7)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


def test_constant_stream_closed_form():
    # one shard of n copies of token 7: every k-context (7,)*k occurs n - k times, always followed by 7
    n = 1000
    train = np.full(n, 7, np.uint16)
    bounds = np.array([0, n], np.int64)
    x = np.full(50, 7, np.uint16)
    tgt = np.full(50, 7, np.uint16)
    avail = O.segments(x)
    for k in (1, 2, 3, 6):
        o = O.query_counts(train, bounds, x, tgt, avail, k, ntop=2)
        valid = avail >= k
        assert np.all(o["tot"][valid] == n - k) and np.all(o["tot"][~valid] == 0)
        assert np.all(o["dist"][valid] == 1) and np.all(o["cnt"][valid] == n - k)
        assert np.all(o["top_tok"][valid, 0] == 7) and np.all(o["top_cnt"][valid, 1] == 0)


def test_shards_do_not_join():
    # "a b" ends shard 0, "c" starts shard 1: the context (a, b) has no next token, (b,) is never followed by c
    a, b, c = 1, 2, 3
    shards = [np.array([a, b], np.uint16), np.array([c, a, b, c], np.uint16)]
    train = np.concatenate(shards)
    bounds = np.array([0, 2, 6], np.int64)
    x = np.array([a, b], np.uint16)
    tgt = np.array([b, c], np.uint16)
    avail = O.segments(x)
    o1 = O.query_counts(train, bounds, x, tgt, avail, 1)
    assert o1["tot"][1] == 1 and o1["cnt"][1] == 1  # (b,) -> c once (shard 1 only)
    o2 = O.query_counts(train, bounds, x, tgt, avail, 2)
    assert o2["tot"][1] == 1 and o2["cnt"][1] == 1  # (a, b) -> c once


def test_ranking_and_top_rule():
    # context (5,) followed by 9 x3, 4 x2, 8 x2, 6 x1: ranks 9, 4, 8, 6 (ties by token ascending)
    seq = [5, 9, 5, 9, 5, 9, 5, 4, 5, 4, 5, 8, 5, 8, 5, 6]
    train = np.array(seq, np.uint16)
    bounds = np.array([0, len(seq)], np.int64)
    x = np.array([5, 5, 5, 5], np.uint16)
    tgt = np.array([9, 4, 8, 6], np.uint16)
    avail = np.array([1, 1, 1, 1], np.int32)
    o = O.query_counts(train, bounds, x, tgt, avail, 1, cnt_top=2, ntop=4)
    assert list(o["top_tok"][0]) == [9, 4, 8, 6] and list(o["top_cnt"][0]) == [3, 2, 2, 1]
    assert list(o["cnt"]) == [3, 2, 0, 0]  # 8 and 6 rank 3rd and 4th: outside cnt_top = 2
    assert o["dist"][0] == 4 and o["tot"][0] == 8


def test_segments_rule():
    x = np.array([3, 4, O.BOS, 5, 6, O.BOS], np.uint16)
    assert list(O.segments(x)) == [1, 2, 1, 2, 3, 1]
    assert list(data.segments(x)) == [1, 2, 1, 2, 3, 1]
    assert list(data.segments(x, breaks=[4])) == [1, 2, 1, 2, 1, 1]


def test_weights_round_half_even():
    c = np.array([[1, 1, 0, 0, 0, 0, 0, 0], [1, 3, 0, 0, 0, 0, 0, 0], [0] * 8], np.uint32)
    w = O.weights(c)
    assert list(w[0, :2]) == [32768, 32768]  # 32767.5 rounds to even
    assert list(w[1, :2]) == [16384, 49151]  # 16383.75, 49151.25
    assert not w[2].any()


def test_deepest_rows_cell_by_hand():
    # one position, variant (2, 3): level 3 matched with total 10 and top count 9 -> bucket 1 (LEVELS.index(3)),
    # count bin #{2,3,5,9 <= 10} = 4, purity 0.9 -> #{.3,.5,.7,.85 <= .9} = 4: ((1+1)*7+4)*6+4 = 112
    per = {}
    for k, tot, top in ((2, 30, 5), (3, 10, 9)):
        o = O._alloc(1, 8)
        o["tot"][0] = tot
        o["top_cnt"][0, :2] = [top, tot - top]
        o["top_tok"][0, :2] = [11, 12]
        per[k] = o
    cell, tokens, w = O.deepest_rows(per, (2, 3))
    assert cell[0] == 112 and list(tokens[0, :2]) == [11, 12]
    assert list(w[0, :2]) == [round(9 / 10 * 65535), round(1 / 10 * 65535)]


def test_features_bins():
    tot = np.array([[0, 1, 2, 3, 1024, 2 ** 31]], np.int64)  # one level
    counts = np.zeros((3, 1, tot.shape[1]), np.int32)
    counts[0, 0] = (tot[0] & 0xFFFFFFFF).astype(np.uint32).view(np.int32)
    counts[1, 0] = [0, 1, 1, 2, 5, 1]
    counts[2, 0] = [0, 1, 3, 1, 0, 7]
    t, d, c, b, s = O.features(counts)
    assert list(b[:, 0]) == [0, 0, 1, 1, 10, 24]  # floor(log2), clamped to 24
    assert list(s[:, 0]) == [25, 26, 26, 25, 25, 26]  # (dist == 1) + 25 * L
    assert list(c[:, 0]) == [0, 1, 2, 1, 0, 7]  # min(cnt, tot)


def test_generator_deterministic_and_shaped():
    a = data.make_corpus("c1", train_tokens=100_000, query_tokens=5_001, shard_tokens=40_000)
    b = data.make_corpus("c1", train_tokens=100_000, query_tokens=5_001, shard_tokens=40_000)
    assert np.array_equal(a.train, b.train) and np.array_equal(a.query, b.query)
    assert len(a.train) == 100_000 and len(a.query) == 5_001
    assert list(a.bounds) == [0, 40_000, 80_000, 100_000]
    assert a.train.max() <= data.BOS
    eos = np.flatnonzero(a.train == data.BOS)
    assert len(eos) > 50  # documents of mean 1025 tokens
    gaps = np.diff(eos)
    assert 500 < gaps.mean() < 2000
    assert len(a.train_plan.copies) > 0 and len(a.query_plan.copies) > 0
    # a copied span of the query stream is a span of the training stream
    dst, src, n = a.query_plan.copies[0]
    assert np.array_equal(a.query[dst : dst + n], a.train[src : src + n])


def test_shard_file_roundtrip(tmp_path):
    t = np.arange(100, dtype=np.uint16)
    p = tmp_path / "s.bin"
    data.write_shard(p, t)
    assert data.shard_tokens(p) == 100
    assert np.array_equal(data.read_shard(p), t)
    bad = tmp_path / "bad.bin"
    bad.write_bytes(b"\0" * 1024)
    with pytest.raises(ValueError):
        data.shard_tokens(bad)


def test_table_rows_by_hand():
    # two positions, row levels (2, 3): position 0 matched level 3 (total 4, counts 3, 1 -> tokens 7, 9), position 1
    # only level 2 (total 40, top 10 of it): entries = 2
    per = {}
    for k, tot, cnts, toks in ((2, (40, 40), (10, 6), (5, 6)), (3, (4, 0), (3, 1), (7, 9))):
        o = O._alloc(2, 8)
        o["tot"][:] = tot
        for i in range(2):
            if tot[i]:
                o["top_cnt"][i, :2] = cnts
                o["top_tok"][i, :2] = toks
        per[k] = o
    cell, nxt, w, level = O.table_rows(per, (2, 3), buckets=(1, 2, 3), entries=2)
    # position 0: bucket 2 (level 3), count bin #{2,3 <= 4} = 2, purity 3/4 = .75 -> #{.3,.5,.7} = 3
    assert cell[0] == ((1 + 2) * 7 + 2) * 6 + 3 and level[0] == 2
    assert list(nxt[0]) == [7, 9] and list(w[0]) == [round(3 / 4 * 65535), round(1 / 4 * 65535)]
    # position 1: bucket 1, count bin 6 (40 >= 33), purity 10/40 = .25 -> 0; weights 10/16, 6/16 of the kept counts
    assert cell[1] == ((1 + 1) * 7 + 6) * 6 + 0 and level[1] == 1
    assert list(w[1]) == [40959, 24576]  # 40959.375, 24575.625


def _online_case(rng, n_parts, part_len, steps):
    shards = [rng.integers(0, 4, size=part_len).astype(np.uint16) for _ in range(n_parts)]
    for sh in shards:
        sh[rng.random(len(sh)) < 0.06] = O.BOS
    tok = np.concatenate(shards)
    bounds = np.cumsum([0] + [len(sh) for sh in shards])
    # spans: each part consumed in `steps` chunks, steps interleaved over the parts
    spans = []
    for j in range(n_parts):
        cuts = np.linspace(bounds[j], bounds[j + 1] - 1, steps + 1).astype(int)
        for s in range(steps):
            if cuts[s] < cuts[s + 1]:
                spans.append((cuts[s], cuts[s + 1], s))
    return tok, bounds, np.array(spans, np.int64)


@pytest.mark.parametrize("seed", range(6))
def test_online_oracle_matches_brute_force(seed):
    rng = np.random.default_rng(300 + seed)
    tok, bounds, spans = _online_case(rng, int(rng.integers(1, 3)), int(rng.integers(30, 70)), int(rng.integers(2, 6)))
    tau, tau_in = O.spans_tau(len(tok), bounds, spans)
    args = (tok, bounds, tau, tau_in, [1, 2, 3], [1, 2, 3, 4], 3, [1, 2, 4], 0, 10)
    got = O.online(*args)
    want = O.brute_online(*args)
    for g, w, name in zip(got, want, ("cell", "next", "weights", "tot", "dist", "cnt", "hinted")):
        assert np.array_equal(g, w), name
    assert got[-1] > 0
    # a sub-range of steps writes only its own queries' rows
    part = O.online(tok, bounds, tau, tau_in, [1, 2, 3], [1, 2, 3, 4], 3, [1, 2, 4], 1, 3)
    part_b = O.brute_online(tok, bounds, tau, tau_in, [1, 2, 3], [1, 2, 3, 4], 3, [1, 2, 4], 1, 3)
    for g, w in zip(part, part_b):
        assert np.array_equal(g, w)


def test_spans_tau():
    # two parts [0, 6), [6, 10); step 0 trains inputs 0..2 (target 3), step 1 inputs 3..5 (target 6 is another part)
    tau, tau_in = O.spans_tau(10, [0, 6, 10], [(0, 3, 0), (3, 6, 1), (6, 9, 0)])
    assert list(tau[:7]) == [0, 0, 0, 0, 1, 1, 0] and tau[9] == 0 and tau_in[3] == 1 and tau_in[9] == O.NONE


def test_features_bins_at_float32_edges():
    """floor(log2) of the float32 total at 2^k - 1: log2(2^k - 1) = k - 2^-k / ln 2 + O(4^-k), and float32 values in
    [16, 32) are 2^-19 apart, so the deficit rounds away (bin k) once 2^-k / ln 2 < 2^-20, i.e. from k = 21 on; below
    that the bin is k - 1. 2^25 - 1 rounds to 2^25 as a float32; bins clamp at 24. torch's own float32 log2 agrees."""
    ks = list(range(18, 26))
    tot = np.array([[(1 << k) - 1 for k in ks] + [(1 << k) for k in ks]], np.int64)
    counts = np.zeros((3, 1, tot.shape[1]), np.int32)
    counts[0, 0] = tot[0].astype(np.uint32).view(np.int32)
    _, _, _, b, _ = O.features(counts)
    want = [k - 1 if k <= 20 else min(k, 24) for k in ks] + [min(k, 24) for k in ks]
    assert list(b[:, 0]) == want
    t = torch.log2(torch.tensor(tot[0].astype(np.float32)))
    assert list(torch.clamp(torch.floor(t), 0, 24).long().tolist()) == want


def test_record_rows_by_hand():
    """build.py:341-387 on hand-made totals and tops (levels 6, 10, 20):
      * position 0: deepest occurring level 10 (tot 3), tops (2, 1) of tokens (7, 9): cell ((1 + 1) * 7 + 2) * 6 + 2
        = 98 (count bin: 2, 3 <= 3; share 2/3: 0.3, 0.5 <= it), entries 7 | 2 << 16, 9 | 1 << 16;
      * position 1: only level 6 (tot 40001), top count 40000 > 32767: weights ceil(c * 32767 / 40000): 32767,
        16384 (for 20000) and 1 (for 1); cell ((1 + 0) * 7 + 6) * 6 + 5 = 83 (share 40000/40001 >= 0.95);
      * position 2: nothing occurred: cell 0, no entries;
      * position 3: level 20 with a top count of 3e9 (row_top clamped to 2^31 - 1, share 0.716 -> purity 3) and
        total 3e9 + 5: cell ((1 + 2) * 7 + 6) * 6 + 3 = 165, weight 32767."""
    tot = np.zeros((3, 4), np.uint32)
    tt = np.zeros((3, 4, 8), np.uint16)
    tc = np.zeros((3, 4, 8), np.uint32)
    tot[:, 0] = [4, 3, 0]
    tt[1, 0, :2], tc[1, 0, :2] = [7, 9], [2, 1]
    tt[0, 0, :1], tc[0, 0, :1] = [7], [4]
    tot[0, 1] = 40001
    tt[0, 1, :3], tc[0, 1, :3] = [5, 6, 8], [40000, 20000, 1]
    tot[:, 3] = [3_000_000_005, 3_000_000_005, 3_000_000_005]
    tt[2, 3, :2], tc[2, 3, :2] = [11, 12], [3_000_000_000, 5]
    cells, entries = O.record_rows(tot, tt, tc)
    assert cells.tolist() == [98, 83, 0, 165]
    assert entries[0, :3].tolist() == [7 | 2 << 16, 9 | 1 << 16, 0]
    assert entries[1, :4].tolist() == [5 | 32767 << 16, 6 | 16384 << 16, 8 | 1 << 16, 0]
    assert not entries[2].any()
    assert entries[3, :2].tolist() == [11 | 32767 << 16, 12 | 1 << 16]


def test_batch_rows_by_hand():
    """build.py:390-403: cells, then (position, entry) pairs of the non-zero entries in position order, padded with
    (i % n, 0); more entries than capacity raise."""
    cells = np.array([5, 0, 7, 9], np.int32)
    entries = np.zeros((4, 8), np.int32)
    entries[0, :2] = [101, 102]
    entries[2, 0] = 103
    entries[3, 1] = 104  # not in the batch below
    rows = O.batch_rows(cells, entries, 0, 3, 5)
    assert rows.tolist() == [5, 0, 7, 0, 101, 0, 102, 2, 103, 0, 0, 1, 0]
    with pytest.raises(AssertionError):
        O.batch_rows(cells, entries, 0, 3, 2)


@pytest.mark.parametrize("seed", range(6))
def test_prefix_rule_drops_no_hit_when_avail_is_closed(seed):
    """The level scans' prefix rule (probe a position only where the previous level hit there and one position
    earlier) on the oracle's own hit sets: with segment-shaped avail every level-k hit has level-(k-1) hits at both."""
    shards, train, bounds, x, tgt = _case(np.random.default_rng(seed), 4, 3, 400, 300)
    avail = O.segments(x)
    prev = None
    for k in range(1, 7):
        h = O.query_counts(train, bounds, x, tgt, avail, k, hits=True)["hits"].astype(bool)
        if prev is not None:
            both = prev.copy()
            both[1:] &= prev[:-1]
            both[0] = False
            assert not (h & ~both).any(), k
            assert h.any() or k > 3, k
        prev = h


def test_prefix_rule_needs_closed_avail():
    """With a hole in avail (query position 1 not answered) the query context (5, 6, 7) of position 2 is indexed
    while its prefix (5, 6) is not: its corpus hit has no level-2 hit one position earlier, so the rule must stay off
    (ng_avail_closed reads such an avail as not closed)."""
    train = np.array([5, 6, 7, 8], np.uint16)
    bounds = np.array([0, 4], np.int64)
    x = np.array([5, 6, 7], np.uint16)
    tgt = np.array([6, 7, 8], np.uint16)
    avail = np.array([1, 0, 3], np.int32)
    h2 = O.query_counts(train, bounds, x, tgt, avail, 2, hits=True)["hits"].astype(bool)
    h3 = O.query_counts(train, bounds, x, tgt, avail, 3, hits=True)["hits"].astype(bool)
    (p,) = np.flatnonzero(h3)
    assert h2[p] and not h2[p - 1]


def test_segment_rule_by_hand():
    """The rule "segment" (online.rs:14-17) on a stream of two segments (the second starts at the BOS at 4): a query
    sees only occurrences whose next token lies before its own segment's start."""
    B = O.BOS
    tok = np.array([5, 6, 5, 6, B, 5, 6, 7], np.uint16)
    cell, nxt, w, tot, dist, cnt, hinted = O.brute_segment(tok, [0, 8], [1], [1, 2], 2, [1, 2])
    # position 5, context (5): occurrences at 0 and 2 (next 6, 6); (B, 5) never occurred before 4
    assert tot[5].tolist() == [2, 0] and dist[5].tolist() == [1, 0] and cnt[5].tolist() == [2, 0]
    # position 6, contexts (6) and (5, 6): the occurrence at 1 (next 5); the one at 3 has its next token at 4
    assert tot[6].tolist() == [1, 1] and dist[6].tolist() == [1, 1] and cnt[6].tolist() == [0, 0]
    # the first segment sees nothing; rows: cell ((1 + 0) * 7 + count bin) * 6 + purity bin
    assert not tot[:5].any() and not tot[7].any()
    assert cell.tolist() == [0, 0, 0, 0, 0, (7 + 1) * 6 + 5, 7 * 6 + 5, 0] and hinted == 2
    assert nxt[5].tolist() == [6, 0] and nxt[6].tolist() == [5, 0]
    assert w[5].tolist() == [65535, 0] and w[6].tolist() == [65535, 0]


@pytest.mark.parametrize("seed", range(6))
def test_segment_rule_is_the_step_rule_over_segments(seed):
    """The GPU's rule "segment" runs the step engine with one step per segment (tau = tau_in = the segment index):
    the step rule's oracle fed those steps equals the segment rule's brute force on random multi-part streams."""
    rng = np.random.default_rng(70 + seed)
    n = int(rng.integers(60, 140))
    tok = rng.integers(0, 3, size=n).astype(np.uint16)
    tok[rng.random(n) < 0.08] = O.BOS
    cuts = sorted(rng.choice(np.arange(10, n - 10), size=int(rng.integers(0, 3)), replace=False).tolist())
    bounds = [0] + cuts + [n]
    starts = np.zeros(n, bool)
    starts[bounds[:-1]] = True
    starts |= tok == O.BOS
    seg = (np.cumsum(starts) - 1).astype(np.uint32)
    args = ([1, 2, 3], [1, 2, 3, 4], 3, [1, 2, 4])
    got = O.online(tok, bounds, seg, seg, *args, 0, int(seg[-1]) + 1)
    want = O.brute_segment(tok, bounds, *args)
    for g, w, name in zip(got, want, ("cell", "next", "weights", "tot", "dist", "cnt", "hinted")):
        assert np.array_equal(g, w), name


def test_train_hints_slots_by_hand():
    """train_hints.rs's slots: a position's deepest levels with a counted occurrence fill its slots, deepest first;
    the hand case's position 6 has both levels, position 5 only level 1, the rest none."""
    B = O.BOS
    tok = np.array([5, 6, 5, 6, B, 5, 6, 7], np.uint16)
    cell, nxt, w, level = O.brute_train_hints(tok, [0, 8], [1, 2], [1, 2], 2, 2)
    assert cell[6].tolist() == [((1 + 1) * 7 + 0) * 6 + 5, (7 + 0) * 6 + 5] and level[6].tolist() == [1, 0]
    assert cell[5].tolist() == [(7 + 1) * 6 + 5, 0] and level[5].tolist() == [0, -1]
    assert nxt[6, :, 0].tolist() == [5, 5] and w[6, :, 0].tolist() == [65535, 65535] and nxt[5, 0, 0] == 6
    others = [0, 1, 2, 3, 4, 7]
    assert not cell[others].any() and (level[others] == -1).all()


def test_loader_plan_by_hand():
    """llm.c's sequential loader plan (hint_stats.cuh loader_plan :395-409) for 2 ranks, B*T = 10, 2 micro-steps
    and 3 steps over shards of 45 and 100 tokens: shard 0 holds (45 - 1) // 20 = 2 samples per rank, then shard 1."""
    from ngram_amd.online import loader_plan, plan_rows, plan_spans, plan_stream

    plan = loader_plan([45, 100], 2, 10, 2, 3)
    rank0 = [(0, 0, 0, 0, 0), (0, 1, 0, 0, 20), (1, 0, 0, 1, 0), (1, 1, 0, 1, 20), (2, 0, 0, 1, 40), (2, 1, 0, 1, 60)]
    rank1 = [(s, m, 1, sh, off + 10) for s, m, _, sh, off in rank0]
    assert [tuple(r) for r in plan] == rank0 + rank1
    sizes = plan_stream([45, 100], plan, 10)
    assert sizes == [45, 81]  # shard 0 whole; shard 1 up to rank 1's last target (70 + 10 + 1)
    spans = plan_spans(plan, sizes, 10)
    assert spans[2].tolist() == [45, 55, 1] and spans[6].tolist() == [10, 20, 0]
    rows = plan_rows(plan, sizes, 10, 2, 1)
    assert rows[:10].tolist() == list(range(10, 20)) and rows[20:30].tolist() == list(range(55, 65))
    with pytest.raises(ValueError):
        loader_plan([45, 100], 2, 10, 2, 4)  # runs past the shards
