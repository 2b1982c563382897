"""GPU: the reference-ABI libraries (gpu_val_stats flavour in libngram_amd.so, record flavour in
libngram_amd_record.so) driven through ctypes as a host binding them does (tests/abi_driver.py), bit-exact against the
CPU oracle: tot / dist / cnt per position and level (the gpu_val_stats flavour with the TOP = 1024 rule, the record's
without), the per-context tops, the variants' hint rows; and the kernels' edge behaviour (count wraps past the packed
count field, owners, grouping, segment bounds at odd offsets)."""

import numpy as np
import pytest
import torch

import abi_driver as D
import oracle as O
from ngram_amd import data
from ngram_amd.build import RECORD_LIB_NAME, lib_path
from ngram_amd.lib import Lib, i32, u64

pytestmark = pytest.mark.gpu

LEVELS = (2, 3, 4, 5, 6, 8, 10, 12, 16, 20)
BUCKETS = (2, 3, 4, 5, 6, 10, 20)
VARIANTS = ((6, 10, 20), (2, 3, 6, 10, 20), BUCKETS)


@pytest.fixture(scope="module")
def corpus():
    return data.make_corpus("c1", train_tokens=600_000, query_tokens=40_001, shard_tokens=250_000)


@pytest.fixture(scope="module")
def dev_corpus(gpu, corpus):
    tok, sizes, starts, L = data.device_tokens(corpus.shards())
    q = corpus.query
    x = torch.from_numpy(q[:-1].view(np.int16).copy()).cuda()
    tgt = torch.from_numpy(q[1:].view(np.int16).copy()).cuda()
    avail = torch.from_numpy(O.segments(q[:-1])).cuda()
    return tok, L, x, tgt, avail


@pytest.fixture(scope="module")
def reference(corpus):
    x, tgt = corpus.query[:-1], corpus.query[1:]
    avail = O.segments(x)
    return {k: O.query_counts(corpus.train, corpus.bounds, x, tgt, avail, k) for k in LEVELS}


@pytest.fixture(scope="module")
def reference_no_top(corpus):
    x, tgt = corpus.query[:-1], corpus.query[1:]
    avail = O.segments(x)
    return {k: O.query_counts(corpus.train, corpus.bounds, x, tgt, avail, k, cnt_top=1 << 30) for k in (2, 3, 4, 6)}


def _libs(flavour):
    return Lib() if flavour == "gvs" else Lib(lib_path(RECORD_LIB_NAME))


def _check_counts(out, reference, levels):
    o = out.cpu().numpy()
    for li, k in enumerate(levels):
        r = reference[k]
        assert np.array_equal(o[0, li].view(np.uint32), r["tot"]), f"tot k={k}"
        assert np.array_equal(o[1, li].astype(np.uint16), r["dist"]), f"dist k={k}"
        assert np.array_equal(o[2, li].view(np.uint32), r["cnt"]), f"cnt k={k}"
        assert (r["tot"] > 0).any()


@pytest.mark.parametrize("how", ["count", "sparse", "emit", "words"])
def test_gvs_flavour_matches_oracle(dev_corpus, reference, how):
    lib = _libs("gvs")
    tok, L, x, tgt, avail = dev_corpus
    out, mask, per = D.level_stats(lib, "gvs", tok, L, x, tgt, avail, LEVELS, how)
    _check_counts(out, reference, LEVELS)
    for variant in VARIANTS:
        rows = D.variant_rows(lib, x.numel(), mask, per, LEVELS, variant, BUCKETS).cpu().numpy()
        cell, tokens, w = O.deepest_rows({k: reference[k] for k in variant}, variant)
        assert np.array_equal(rows, O.pack_rows(cell, tokens, w)), f"rows {variant}"


@pytest.mark.parametrize("how", ["count", "sparse", "emit", "words"])
def test_record_flavour_matches_oracle(dev_corpus, reference_no_top, how):
    lib = _libs("rec")
    tok, L, x, tgt, avail = dev_corpus
    levels = (2, 3, 4, 6)
    out, _, per = D.level_stats(lib, "rec", tok, L, x, tgt, avail, levels, how, top=4, cnt_top=0)
    _check_counts(out, reference_no_top, levels)
    # the ranked tops per position (pos_topk, the record library's extension) against the oracle's top-4
    for li, k in enumerate(levels):
        qt, top_tok, top_cnt, _, _ = per[k]
        N = x.numel()
        ot = torch.zeros((N, 4), dtype=torch.int16, device=x.device)
        oc = torch.zeros((N, 4), dtype=torch.int32, device=x.device)
        lib("pos_topk", qt.ctx_of, N, 0, qt.ids, top_tok, top_cnt, i32(4), i32(4), ot, oc)
        r = reference_no_top[k]
        assert np.array_equal(ot.cpu().numpy().view(np.uint16), r["top_tok"][:, :4]), f"top tokens k={k}"
        assert np.array_equal(oc.cpu().numpy().view(np.uint32), r["top_cnt"][:, :4]), f"top counts k={k}"


@pytest.mark.parametrize("flavour", ["gvs", "rec"])
def test_overflowing_table_reruns(dev_corpus, reference, flavour):
    """A pair table far too small overflows (flags[0]); the driver doubles it and scans again, exactly."""
    lib = _libs(flavour)
    tok, L, x, tgt, avail = dev_corpus
    out, _, per = D.level_stats(lib, flavour, tok, L, x, tgt, avail, (2, 3), "count", cap=256,
                                cnt_top=1024 if flavour == "gvs" else 0)
    assert per[2][4] > 0
    if flavour == "gvs":
        _check_counts(out, reference, (2, 3))


@pytest.mark.parametrize("flavour,cb", [("gvs", 24), ("rec", 23)])
def test_aggregate_counts_past_the_count_field(gpu, flavour, cb):
    """One pair key counted 2^cb + 1000 times (past the packed slot's count field: the wrap byte carries) among a few
    others; part_scatter returns the exact counts."""
    lib = _libs(flavour)
    hot, n_hot = (5 << 16) | 77, (1 << cb) + 1000
    others = torch.tensor([(1 << 16) | 3, (2 << 16) | 9, (9 << 16) | 1], dtype=torch.int64, device="cuda")
    keys = torch.cat([torch.full((n_hot,), hot, dtype=torch.int64, device="cuda"), others.repeat(7)])
    keys = keys[torch.randperm(keys.numel(), device="cuda")]
    n, pbits, sub_cap = keys.numel(), 2, 64
    counts = torch.zeros(1 << pbits, dtype=torch.int64, device="cuda")
    lib("subpart_count", keys, n, i32(pbits), counts)
    grouped = torch.empty_like(keys)
    cursor = torch.cumsum(counts, 0) - counts
    lib("subpart_scatter", keys, n, i32(pbits), cursor, grouped)
    cap = sub_cap << pbits
    pk = torch.full((cap,), -1, dtype=torch.int64, device="cuda")
    wraps = torch.zeros(cap // 4, dtype=torch.int32, device="cuda")
    flags = torch.zeros(2, dtype=torch.int32, device="cuda")
    lib("aggregate", grouped, n, pk, wraps, u64(sub_cap), i32(pbits), flags, i32(0))
    assert int(flags[0].item()) == 0
    k, v, _ = D.drain(lib, pk, wraps, cap, [0, 16])
    got = dict(zip(k.cpu().tolist(), v.cpu().numpy().view(np.uint32).tolist()))
    want = {hot: n_hot, **{int(o): 7 for o in others.cpu()}}
    assert got == want


def test_drain_by_owner(gpu):
    """part_count / part_scatter with three owners: every entry in its owner's run, counts exact."""
    lib = _libs("gvs")
    g = torch.Generator(device="cpu").manual_seed(5)
    ctx = torch.randint(0, 3000, (20000,), generator=g)
    nxt = torch.randint(0, 50000, (20000,), generator=g)
    keys = ((ctx << 16) | nxt).cuda()
    flat = torch.zeros(1, dtype=torch.int64, device="cuda")
    cap, pbits = 1 << 16, 0
    pk = torch.full((cap,), -1, dtype=torch.int64, device="cuda")
    wraps = torch.zeros(cap // 4, dtype=torch.int32, device="cuda")
    flags = torch.zeros(2, dtype=torch.int32, device="cuda")
    lib("aggregate", keys, keys.numel(), pk, wraps, u64(cap), i32(pbits), flags, i32(0))
    del flat
    bounds = [0, 700, 2100, 3000]
    k, v, per = D.drain(lib, pk, wraps, cap, bounds)
    uk, uc = torch.unique(keys.cpu(), return_counts=True)
    assert sorted(zip(k.cpu().tolist(), v.cpu().tolist())) == sorted(zip(uk.tolist(), uc.tolist()))
    c = (k.cpu() >> 16).numpy()
    runs = np.cumsum([0] + per.cpu().tolist())
    for o in range(3):
        part = c[runs[o] : runs[o + 1]]
        assert ((part >= bounds[o]) & (part < bounds[o + 1])).all()


def test_owner_side_at_odd_offsets(gpu):
    """seg_bounds, ctx_tot, rank_keys and rank_scatter on views that start at an odd element (the kernels' scalar
    paths) agree with numpy."""
    lib = _libs("gvs")
    rng = np.random.default_rng(3)
    ctx = np.sort(rng.integers(0, 500, 7001))
    tokn = rng.integers(0, 60000, 7001)
    keys = np.unique((ctx.astype(np.int64) << 16) | tokn)
    cnt = rng.integers(1, 50, len(keys)).astype(np.int32)
    U, ids = len(keys), 500
    uk_full = torch.from_numpy(np.r_[0, keys]).cuda()
    ag_full = torch.from_numpy(np.r_[0, cnt]).cuda()
    uk, agg = uk_full[1:], ag_full[1:]
    start = torch.zeros(ids, dtype=torch.int64, device="cuda")
    end = torch.zeros(ids, dtype=torch.int64, device="cuda")
    lib("seg_bounds", uk, U, start, end)
    c = keys >> 16
    present = np.unique(c)
    s_np = np.searchsorted(c, present, "left")
    e_np = np.searchsorted(c, present, "right")
    assert np.array_equal(start.cpu().numpy()[present], s_np) and np.array_equal(end.cpu().numpy()[present], e_np)
    tot = torch.empty(ids, dtype=torch.int64, device="cuda")
    lib("ctx_tot", start, end, agg, ids, tot)
    assert np.array_equal(tot.cpu().numpy()[present], np.add.reduceat(cnt.astype(np.int64), s_np))
    k2 = torch.empty(U + 1, dtype=torch.int64, device="cuda")[1:]
    v2 = torch.empty(U + 1, dtype=torch.int32, device="cuda")[1:]
    lib("rank_keys", uk, agg, U, k2, v2)
    k2s, sv = torch.empty_like(k2), torch.empty_like(v2)
    lib.cub("sort_pairs", k2, k2s, v2, sv, U, i32(0), i32(41))
    rank_of = torch.empty(U, dtype=torch.int32, device="cuda")
    top_tok = torch.zeros(ids * 8, dtype=torch.int16, device="cuda")
    top_cnt = torch.zeros(ids * 8, dtype=torch.int32, device="cuda")
    lib("rank_scatter", sv, U, uk, agg, start, rank_of, top_tok, top_cnt, i32(8))
    order = np.lexsort((keys & 0xFFFF, -cnt, c))
    rank = np.empty(U, np.int64)
    rank[order] = np.arange(U) - s_np[np.searchsorted(present, c[order])]
    assert np.array_equal(rank_of.cpu().numpy(), rank)
    tt = top_tok.cpu().numpy().view(np.uint16).reshape(ids, 8)
    for p in present[:50]:
        sel = order[c[order] == p][:8]
        assert np.array_equal(tt[p, : len(sel)], (keys[sel] & 0xFFFF).astype(np.uint16))


def test_val_keys_group_equal_contexts(gpu):
    """val_keys: EMPTY where the context does not fit its segment, equal keys exactly for equal contexts (k = 3 is
    exact; k = 7 hashed, no collision expected at this size)."""
    lib = _libs("gvs")
    rng = np.random.default_rng(1)
    q = rng.integers(0, 40, 30000).astype(np.uint16)
    q[rng.random(30000) < 0.01] = data.BOS
    avail = O.segments(q)
    x = torch.from_numpy(q.view(np.int16)).cuda()
    av = torch.from_numpy(avail).cuda()
    for k in (3, 7):
        keys = torch.empty(len(q), dtype=torch.int64, device="cuda")
        lib("val_keys", x, av, len(q), i32(k), keys)
        kk = keys.cpu().numpy()
        valid = avail >= k
        assert np.array_equal(kk != -1, valid)
        ctx = np.lib.stride_tricks.sliding_window_view(np.r_[np.zeros(k - 1, np.uint16), q], k)
        pairs = {}
        for i in np.flatnonzero(valid):
            pairs.setdefault(ctx[i].tobytes(), set()).add(int(kk[i]))
        assert all(len(v) == 1 for v in pairs.values())
        assert len({next(iter(v)) for v in pairs.values()}) == len(pairs)
