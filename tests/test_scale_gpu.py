"""GPU: parity at each BASELINE configuration's stated size, bit-exact against the CPU oracle.

  * c1 whole: 4M training + 256K query tokens, k = 2, 3: tot / dist / cnt, the top-1 next token and its count, the
    longest match (cap 32);
  * c2 whole: CountTable over 100M tokens, n = 2..4, 8M query positions, tot / dist / cnt and the top-4;
  * c3 sampled: the build over the whole 1B-token corpus for 16M query positions (n = 2..8, top-4); at least 100K of
    its positions compared with the oracle run over the whole corpus: random windows, the positions of the hottest
    level-2 contexts, and level-3 positions whose context id is at least 2^25 (the packed words' 26-bit ids);
  * c4 whole: the 92 online steps of 2^19 tokens, every hint and count row;
  * c5 sampled: the longest match (cap 64) of 16M positions of a 64M-token held-out stream against the 1B corpus,
    at least 100K of them compared with the oracle over the whole corpus.
A sample is a set of windows of consecutive query positions with the positions before them kept as context (their
avail set to 0, so the oracle counts only the compared positions)."""

import numpy as np
import pytest
import torch

import oracle as O
from ngram_amd import data

pytestmark = pytest.mark.gpu


def _windows(starts: np.ndarray, lead: int, width: int, n: int, av: np.ndarray, keep=None):
    """Query positions of windows [s, s + width) with `lead` context positions before each: (index into the stream,
    avail of the sample (0 on lead positions and on positions not kept), the compared mask)."""
    starts = np.unique(np.clip(starts, lead, n - width))
    idx = (starts[:, None] + np.arange(-lead, width)[None, :]).reshape(-1)
    off = np.tile(np.arange(-lead, width), len(starts))
    cmp = off >= 0
    if keep is not None:
        cmp &= keep[idx]
    avail = np.where(cmp, av[idx], 0).astype(np.int32)
    return idx, avail, cmp


def test_c1_whole(gpu):
    from ngram_amd.counts import CountBuild, queries
    from ngram_amd.lib import Lib
    from ngram_amd.longest import _segments, longest_match

    c = data.make_corpus("c1")
    cb = CountBuild(c.shards(), levels=(2, 3), level_shards={}, topk=1)
    cb.start_load(1)
    x, tgt, avail = queries(c.query, [], "cuda")
    out = cb.counts(x, tgt, avail).cpu().numpy()
    xs, ts = c.query[:-1], c.query[1:]
    av = O.segments(xs)
    for li, k in enumerate((2, 3)):
        o = O.query_counts(c.train, c.bounds, xs, ts, av, k, cnt_top=1 << 30, ntop=1)
        assert np.array_equal(out[0, li].view(np.uint32), o["tot"]) and np.array_equal(out[2, li].view(np.uint32),
                                                                                        o["cnt"]), k
        assert np.array_equal(out[1, li].astype(np.uint16), o["dist"]), k
        assert np.array_equal(cb.top_tok[li, :, 0].cpu().numpy().view(np.uint16), o["top_tok"][:, 0]), k
        assert np.array_equal(cb.top_cnt[li, :, 0].cpu().numpy().view(np.uint32), o["top_cnt"][:, 0]), k
    tok, _, _, _ = data.device_tokens(c.shards())
    length, nxt, cnt, _ = longest_match(tok, x, _segments(x, Lib()), 32)
    want = O.longest_match(c.train, c.bounds, xs, av, 32)
    assert np.array_equal(length.cpu().numpy().view(np.uint32), want[0])
    assert np.array_equal(nxt.cpu().numpy().view(np.uint16), want[1])
    assert np.array_equal(cnt.cpu().numpy().view(np.uint32), want[2])
    assert want[0].max() == 32


def test_c2_whole(gpu):
    from ngram_amd.count_table import CountTable, _segments_device

    dc = data.device_corpus("c2")
    levels = list(dc.config.levels)
    ct = CountTable.from_device(dc.tok, dc.sizes, dc.starts, levels)
    ct.build()
    x, tgt = dc.query[:-1], dc.query[1:]
    res = ct.query_device(x, tgt, _segments_device(x, ct.lib), topk=4)
    train = dc.flat.cpu().numpy().view(np.uint16)
    q = dc.query.cpu().numpy().view(np.uint16)
    xs, ts = q[:-1], q[1:]
    av = O.segments(xs)
    c = res["counts"].cpu().numpy()
    tt, tc = res["top_tok"].cpu().numpy().view(np.uint16), res["top_cnt"].cpu().numpy().view(np.uint32)
    for li, k in enumerate(levels):
        o = O.table_counts(train, dc.bounds, xs, ts, av, k, ntop=4)
        assert np.array_equal(c[0, li].view(np.uint32), o["tot"]) and np.array_equal(c[2, li].view(np.uint32),
                                                                                      o["cnt"]), k
        assert np.array_equal(c[1, li].astype(np.uint16), o["dist"]), k
        assert np.array_equal(tt[li], o["top_tok"]) and np.array_equal(tc[li], o["top_cnt"]), k
    assert len(train) == 100_000_000 and len(xs) == 8_000_000


def test_c3_sampled_over_the_whole_corpus(gpu):
    from ngram_amd.counts import CountBuild, device_queries

    dc = data.device_corpus("c3")
    levels = dc.config.levels
    cb = CountBuild.from_device(dc.tok, dc.sizes, dc.starts, levels=levels, level_shards={}, topk=4)
    x, tgt, avail = device_queries(dc.query)
    res = cb.engine.build(x, tgt, avail, topk=4, keep=(3,))
    N = x.numel()
    ctx3 = res.kept[3][0].cpu().numpy()
    out = res.counts.cpu().numpy()
    top_tok = res.top_tok.cpu().numpy().view(np.uint16)
    top_cnt = res.top_cnt.cpu().numpy().view(np.uint32)
    del res, cb
    rng = np.random.default_rng(33)
    av = avail.cpu().numpy()
    hot = np.argsort(out[0, 0].view(np.uint32))[-300:]  # the positions of the hottest level-2 contexts
    wide = np.flatnonzero(ctx3 >= 1 << 25)
    assert len(wide) > 1000, "level 3 uses context ids of 26 bits"
    wide = rng.choice(wide, 300, replace=False)
    starts = np.concatenate([rng.integers(0, N, 1600), hot - 32, wide - 32])
    idx, s_av, cmp = _windows(starts, 7, 64, N, av)
    assert cmp.sum() >= 100_000
    assert (ctx3[idx[cmp]] >= 1 << 25).sum() >= 300
    q = dc.query.cpu().numpy().view(np.uint16)
    xs, ts = q[:-1][idx], q[1:][idx]
    train = dc.flat.cpu().numpy().view(np.uint16)
    del dc
    torch.cuda.empty_cache()
    gate = None
    for li, k in enumerate(levels):
        o = O.query_counts(train, np.array(_bounds(train), np.int64), xs, ts, s_av, k,
                           cnt_top=1 << 30, ntop=4, hits=True, gate=gate)
        gate = o["hits"]
        g = idx[cmp]
        assert np.array_equal(out[0, li, g].view(np.uint32), o["tot"][cmp]), f"tot k={k}"
        assert np.array_equal(out[1, li, g].astype(np.uint16), o["dist"][cmp]), f"dist k={k}"
        assert np.array_equal(out[2, li, g].view(np.uint32), o["cnt"][cmp]), f"cnt k={k}"
        assert np.array_equal(top_tok[li, g], o["top_tok"][cmp]), f"top_tok k={k}"
        assert np.array_equal(top_cnt[li, g], o["top_cnt"][cmp]), f"top_cnt k={k}"
        if k == 3:
            sel = cmp & (ctx3[idx] >= 1 << 25)
            assert (o["tot"][sel] > 0).any(), "26-bit ids with occurrences"


def _bounds(train: np.ndarray) -> list[int]:
    """The c3 corpus' shard bounds (shards of the configuration's shard size)."""
    return data.train_bounds(len(train), data.CONFIGS["c3"].shard_tokens).tolist()


def test_c5_sampled_over_the_whole_corpus(gpu):
    from ngram_amd.lib import Lib
    from ngram_amd.longest import _segments, longest_match

    print("c5: corpus", flush=True)
    dc = data.device_corpus("c3", query_tokens=1001)
    zipf = dc.zipf
    n = 64_000_000 + 1
    qp = data.make_plan(data.stream_key("c5", "query", n), n, copy_rate=0.15, copy_len=(16, 2048), source=dc.train_plan)
    print("c5: corpus generated", flush=True)
    q = data.realize_gpu(qp, zipf, Lib(), source=dc.flat)
    x = q[:-1]
    avail = _segments(x, Lib())
    torch.cuda.synchronize()
    print("c5: held-out stream generated", flush=True)
    query = torch.zeros(x.numel(), dtype=torch.bool, device=x.device)
    query[3::4] = True
    length, nxt, cnt, _ = longest_match(dc.tok, x, avail, 64, query=query)
    length, nxt, cnt = (t.cpu().numpy() for t in (length, nxt, cnt))
    print("c5: GPU longest match done", flush=True)
    N = x.numel()
    rng = np.random.default_rng(55)
    av = avail.cpu().numpy()
    keep = np.zeros(N, bool)
    keep[3::4] = True
    long_ones = np.flatnonzero(keep & (length >= 40))
    starts = np.concatenate([rng.integers(0, N, 6000), rng.choice(long_ones, min(300, len(long_ones)), False) - 32])
    idx, s_av, cmp = _windows(starts, 63, 64, N, av, keep)
    assert cmp.sum() >= 100_000
    xs = x.cpu().numpy().view(np.uint16)[idx]
    train = dc.flat.cpu().numpy().view(np.uint16)
    del dc, q, x
    torch.cuda.empty_cache()
    print(f"c5: oracle over {len(train)} corpus tokens, {len(xs)} query positions", flush=True)
    want = O.longest_match(train, np.array(_bounds(train), np.int64), xs, s_av, 64)
    g = idx[cmp]
    assert np.array_equal(length[g].view(np.uint32), want[0][cmp])
    assert np.array_equal(nxt[g].view(np.uint16), want[1][cmp])
    assert np.array_equal(cnt[g].view(np.uint32), want[2][cmp])
    assert want[0][cmp].max() == 64


def test_c4_whole_stream(gpu):
    from ngram_amd.lib import Lib
    from ngram_amd.online import OnlineRows

    zipf, plan, spans = data.c4_stream()
    tok = data.realize_gpu(plan, zipf, Lib()).cpu().numpy().view(np.uint16)
    n = len(tok)
    levels, buckets = [2, 3, 4, 5, 6], [2, 3, 4, 5, 6, 10, 20]
    rows = OnlineRows(tok, [0, n], spans)
    got = (np.zeros(n, np.int16), np.zeros((n, 8), np.uint16), np.zeros((n, 8), np.uint16),
           np.zeros((n, 5), np.uint32), np.zeros((n, 5), np.uint16), np.zeros((n, 5), np.uint32))
    hinted = rows.advance(len(spans), levels, buckets, 8, levels, *got)
    tau, tau_in = O.spans_tau(n, [0, n], spans)
    want = O.online(tok, [0, n], tau, tau_in, levels, buckets, 8, levels, 0, len(spans))
    for g, w, name in zip(got, want, ("cell", "next", "weights", "tot", "dist", "cnt")):
        assert np.array_equal(g, w), name
    assert hinted == want[-1] and n == 92 * (1 << 19)
