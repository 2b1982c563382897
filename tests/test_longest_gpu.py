"""GPU: the longest exact suffix match (ngram_amd.longest, configuration c5) against the oracle's
restatement (oracle_longest_match, pinned by brute force on tiny streams): length, next token, its count."""

import numpy as np
import pytest
import torch

import oracle as O
from ngram_amd import data
from ngram_amd.data import device_tokens as load_shards
from ngram_amd.lib import Lib, i32
from ngram_amd.longest import LongestMatch, _segments, longest_match

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def corpus():
    # held-out queries with 15% of documents carrying copied spans of 16-2048 training tokens: long matches
    return data.make_corpus("c5", train_tokens=700_000, query_tokens=60_001, shard_tokens=300_000)


@pytest.mark.parametrize("cap,seg,count", [(64, False, "32"), (64, True, "64"), (8, False, "32overfull"),
                                           (1, True, "64"), (64, False, "64")])
def test_longest_match_matches_oracle(corpus, cap, seg, count, monkeypatch):
    """count: the bitmap levels' final contexts counted by the 32-bit count (32; 32overfull: partitions declared
    overfull at 64 distinct pairs, so levels are counted again with more partition bits, or by the 64-bit count once
    there are none) or by the 64-bit count (64)."""
    import ngram_amd.longest as LG
    from ngram_amd import partcount as P

    monkeypatch.setattr(LG, "_WIDE", set())
    if seg:  # the bitmap levels' counts read the scan regions directly however few events they hold
        monkeypatch.setattr(P, "SEG_MIN_EVENTS", 0)
    if count == "64":
        monkeypatch.setattr(LG, "W_MAX", 0)
    if count == "32overfull":
        monkeypatch.setattr(P, "P32_LIMIT", 64)
    x = corpus.query[:-1]
    avail = O.segments(x)
    want = O.longest_match(corpus.train, corpus.bounds, x, avail, cap)
    tok, sizes, starts, L = load_shards(corpus.shards())
    xt = torch.from_numpy(x.view(np.int16).copy()).cuda()
    av = _segments(xt, Lib())
    assert np.array_equal(av.cpu().numpy(), avail)
    length, nxt, cnt, ladder = longest_match(tok, xt, av, cap)
    got = (length.cpu().numpy().view(np.uint32), nxt.cpu().numpy().view(np.uint16), cnt.cpu().numpy().view(np.uint32))
    for g, w, name in zip(got, want, ("length", "next", "count")):
        assert np.array_equal(g, w), name
    assert want[0].max() == cap  # the copies reach the cap
    # the ladder's matched counts are the positions whose length reaches k
    for k, eligible, matched in ladder:
        assert matched == int((want[0] >= k).sum()) and eligible == int((avail >= k).sum())


@pytest.mark.parametrize("every", [40, 64])
def test_deep_levels_where_no_position_reaches_the_cap(corpus, every):
    """A segment start every `every` tokens keeps every match below the cap of 64 (avail < 64), while the copies
    still run the deep levels: the round at the cap finds nothing and the levels in between carry every position."""
    x = corpus.query[:-1].copy()
    x[::every] = O.BOS
    avail = O.segments(x)
    want = O.longest_match(corpus.train, corpus.bounds, x, avail, 64)
    assert 20 < want[0].max() < 64
    tok, sizes, starts, L = load_shards(corpus.shards())
    xt = torch.from_numpy(x.view(np.int16).copy()).cuda()
    length, nxt, cnt, ladder = longest_match(tok, xt, _segments(xt, Lib()), 64)
    got = (length.cpu().numpy().view(np.uint32), nxt.cpu().numpy().view(np.uint16), cnt.cpu().numpy().view(np.uint32))
    for g, w, name in zip(got, want, ("length", "next", "count")):
        assert np.array_equal(g, w), name
    assert len(ladder) == int(want[0].max()) or ladder[-1][2] == 0
    for k, eligible, matched in ladder:
        assert matched == int((want[0] >= k).sum()) and eligible == int((avail >= k).sum())


def test_device_levels_match_host_levels(corpus, monkeypatch):
    """The existence phase's deep levels run as one stream of launches (no host sync) or level by level on the host:
    the same lengths, next tokens, counts and ladder."""
    from ngram_amd import longest as LG

    x = corpus.query[:-1]
    tok, sizes, starts, L = load_shards(corpus.shards())
    xt = torch.from_numpy(x.view(np.int16).copy()).cuda()
    av = _segments(xt, Lib())
    got = {}
    for dev_levels in (True, False):
        monkeypatch.setattr(LG, "DEVICE_LEVELS", dev_levels)
        length, nxt, cnt, ladder = longest_match(tok, xt, av, 64)
        got[dev_levels] = (length.cpu(), nxt.cpu(), cnt.cpu(), ladder)
    for a, b in zip(got[True][:3], got[False][:3]):
        assert torch.equal(a, b)
    assert got[True][3] == got[False][3] and len(got[True][3]) == 64


def test_unchecked_index_that_overflowed_counts_its_batch_again(corpus, monkeypatch):
    """The list levels' query indexes are built without a host wait and checked once, with their batch's event
    total. One that reports an insert without a slot (forced here from the host, on an index that is in fact whole)
    makes the batch count again on indexes checked as they are built: the same outputs."""
    from ngram_amd import longest as LG

    x = corpus.query[:-1]
    tok, sizes, starts, L = load_shards(corpus.shards())
    xt = torch.from_numpy(x.view(np.int16).copy()).cuda()
    av = _segments(xt, Lib())
    want = longest_match(tok, xt, av, 64)
    flagged = []

    class Flagged(LG.QueryIndex):
        def __init__(self, *a, **kw):
            super().__init__(*a, **kw)
            if kw.get("defer") and self.n is None:
                self.pending[1] = 1
                flagged.append(a[3])

    monkeypatch.setattr(LG, "QueryIndex", Flagged)
    got = longest_match(tok, xt, av, 64)
    assert len(flagged) > 10
    for g, w in zip(got[:3], want[:3]):
        assert torch.equal(g, w)


def test_ladder_interface(corpus, tmp_path):
    paths, _ = corpus.write(tmp_path)
    lm = LongestMatch.create(paths, corpus.query[:20_001], 4, [])
    t = lm.build()
    assert t["total"] > 0 and t["levels"] >= 1
    x = corpus.query[:20_000]
    want = O.longest_match(corpus.train, corpus.bounds, x, O.segments(x), 64)
    assert np.array_equal(lm.length, want[0]) and np.array_equal(lm.next, want[1]) and np.array_equal(lm.count, want[2])
    with pytest.raises(ValueError):
        LongestMatch.create(paths, np.array([3], np.uint16))


def test_context_hint_from_a_much_smaller_call():
    """The longest match sizes each level's query index from the last call's contexts per position: after a call of
    a few contexts repeated, a call over varied text gets tables sized far too small from that hint; an insert gives
    up after a bounded walk and the index is rebuilt at its positions' size, and the result is a first call's."""
    from ngram_amd import longest as LM
    from ngram_amd.lib import Lib

    c = data.make_corpus("c3", train_tokens=600_000, query_tokens=200_001, shard_tokens=300_000)
    tok, _, _, _ = data.device_tokens(c.shards())
    x = torch.from_numpy(c.query[:-1].view(np.int16)).cuda()
    LM._CONTEXTS.clear()
    want = LM.longest_match(tok, x, LM._segments(x, Lib()), 32)
    small = x[:100].repeat(50)  # 5000 positions, about 100 contexts per level: a hint 30 times too small
    LM.longest_match(tok, small, LM._segments(small, Lib()), 32)
    assert LM._CONTEXTS[2] < 0.05
    got = LM.longest_match(tok, x, LM._segments(x, Lib()), 32)
    for g, w in zip(got[:3], want[:3]):
        assert torch.equal(g, w)


@pytest.mark.parametrize("seed,grid", [(3, 2048), (4, 7)])
def test_level_one_scan_by_token(seed, grid):
    """ng_scan_tok1 (level 1 with the token as the context id) against numpy: position p hits where tok[p - 1] is a
    query token and neither it nor tok[p] is SENT; the hit bitmap, the tokens that occurred and each hit's id. The
    corpus starts and ends with SENT and holds SENT runs; a few blocks (grid 7) walk many rounds each."""
    rng = np.random.default_rng(seed)
    L = 32 * 3001
    tok = rng.zipf(1.3, L).clip(1, 60000).astype(np.uint16)
    tok[rng.random(L) < 0.02] = 0xFFFF
    tok[:3] = 0xFFFF
    tok[-5:] = 0xFFFF
    query = np.unique(np.concatenate([rng.integers(0, 60000, 300), tok[rng.integers(0, L, 500)]])).astype(np.uint16)
    query = query[query != 0xFFFF]
    member = np.zeros(65536, bool)
    member[query] = True
    words = np.packbits(member.reshape(-1, 32)[:, ::-1], axis=1).view(">u4").astype(np.uint32).reshape(-1)
    prev = np.concatenate([[0xFFFF], tok[:-1]]).astype(np.int64)
    want_hit = (prev != 0xFFFF) & (tok != 0xFFFF) & member[prev]
    want_bm = np.packbits(want_hit.reshape(-1, 32)[:, ::-1], axis=1).view(">u4").astype(np.uint32).reshape(-1)
    occurred = np.zeros(65536, bool)
    occurred[prev[want_hit]] = True
    want_tokhit = np.packbits(occurred.reshape(-1, 32)[:, ::-1], axis=1).view(">u4").astype(np.uint32).reshape(-1)

    lib = Lib()
    d_tok = torch.from_numpy(tok.view(np.int16)).cuda()
    d_member = torch.from_numpy(words.view(np.int32)).cuda()
    bm = torch.full((L // 32,), -1, dtype=torch.int32, device="cuda")  # every word written: no fill needed
    hit = torch.zeros(2048, dtype=torch.int32, device="cuda")
    ids = torch.full((L,), -7, dtype=torch.int32, device="cuda")
    lib("ng_scan_tok1", d_tok, L, d_member, bm, hit, ids, i32(grid))
    torch.cuda.synchronize()
    assert np.array_equal(bm.cpu().numpy().view(np.uint32), want_bm)
    assert np.array_equal(hit.cpu().numpy().view(np.uint32), want_tokhit)
    got_ids = ids.cpu().numpy()
    assert np.array_equal(got_ids[want_hit], prev[want_hit])
    assert (got_ids[~want_hit] == -7).all()  # positions without a hit are left as they are
    # without an ids array (the counting scan then reads the token before each hit): the same bitmap and tokens
    bm2 = torch.full((L // 32,), -1, dtype=torch.int32, device="cuda")
    hit2 = torch.zeros(2048, dtype=torch.int32, device="cuda")
    lib("ng_scan_tok1", d_tok, L, d_member, bm2, hit2, None, i32(grid))
    torch.cuda.synchronize()
    assert torch.equal(bm2, bm) and torch.equal(hit2, hit)
    with pytest.raises(RuntimeError):
        lib("ng_scan_tok1", d_tok, L - 1, d_member, bm, hit, ids, i32(grid))  # L not a multiple of 32
