"""GPU: the record's surface (CountBuild, record_367_gpu_counts/track_1_short/counts/build.py, on the engine's level
pipeline) bit-exact against the CPU oracle on seeded synthetic streams: per level tot / dist / cnt (no TOP rule), the
top-4 next tokens, the record's rows and batch_rows; the partitioned count's variants (repartitioning, the escape
table, the scans' listing modes, the regions read directly)."""

import numpy as np
import pytest
import torch

import oracle as O
from ngram_amd import counts as C
from ngram_amd import data
from ngram_amd import levels as levels_mod
from ngram_amd import partcount as P

pytestmark = pytest.mark.gpu

LEVELS = (2, 3, 4, 5, 6, 10, 20)


@pytest.fixture(scope="module")
def corpus():
    return data.make_corpus("c3", train_tokens=700_000, query_tokens=50_001, shard_tokens=250_000)


def _reference(corpus, levels, level_shards, ntop=8):
    x, tgt = corpus.query[:-1], corpus.query[1:]
    avail = O.segments(x)
    ref = {}
    nshards = len(corpus.bounds) - 1
    for k in levels:
        m = min(nshards, level_shards.get(k, nshards))
        b = corpus.bounds[: m + 1]
        ref[k] = O.query_counts(corpus.train[: b[-1]], b, x, tgt, avail, k, cnt_top=1 << 30, ntop=ntop)
    return ref


@pytest.mark.parametrize("level_shards,mode", [({}, "part"), ({2: 1, 3: 2}, "part"), ({}, "compact"),
                                               ({2: 1, 3: 2}, "regroup"), ({}, "escape"), ({}, "seg"),
                                               ({2: 1, 3: 2}, "seg"), ({}, "list"), ({2: 1, 3: 2}, "list"),
                                               ({}, "regroup32"), ({2: 1, 3: 2}, "escape32"), ({}, "wide")])
def test_counts_match_oracle(corpus, level_shards, mode, monkeypatch):
    """Modes: the 32-bit count (part, compact, list; regroup32: partitions overfull at 64 distinct pairs, so each
    level is counted again with one more partition bit until none is; escape32: an 8-bit count field, larger counts in
    the escape table; wide: that table too small, so the level is counted again by the 64-bit path) and the 64-bit
    path (regroup, escape, seg: W_MAX 0 sends every level there)."""
    if mode in ("regroup", "escape", "seg"):
        monkeypatch.setattr(P, "W_MAX", 0)
        monkeypatch.setattr(levels_mod, "W_MAX", 0)
    if mode == "regroup32":
        monkeypatch.setattr(P, "P32_LIMIT", 64)
    if mode in ("escape32", "wide"):
        monkeypatch.setattr(P, "PACK32_MIN_BITS", 40)
    if mode == "wide":
        monkeypatch.setattr(P, "ESC_CAP", 16)
    if mode == "regroup":
        # one partition per level to start with: each level's LDS table overflows and it is repartitioned bit by bit;
        # three blocks, each counting a run of partitions
        monkeypatch.setattr(P, "PART_TARGET", 1 << 30)
        monkeypatch.setattr(P, "PART_MIN_BITS", 0)
        monkeypatch.setattr(P, "PART_BLOCKS", 3)
    if mode == "seg":  # the partition sort's first pass reads the scan regions however few events they hold
        monkeypatch.setattr(P, "SEG_MIN_EVENTS", 0)
    if mode == "escape":  # an 8-bit count field: counts of 255 and more go to the escape table
        monkeypatch.setattr(P, "PACK_MIN_BITS", 40)
    cb = C.CountBuild(corpus.shards(), levels=LEVELS, level_shards=level_shards, topk=4)
    if mode in ("compact", "list"):
        # every gated level scans its LDS-listed set positions, or (list) the positions listed in memory first
        cb.engine.density = {k: 0.0 for k in LEVELS}
        if mode == "compact":
            monkeypatch.setattr(levels_mod, "LIST_DENSITY", 0.0)
    cb.start_load(3)
    with pytest.raises(ValueError):
        cb.load_ms()  # a share of the copies is still pending
    cb.pace()
    cb.pace()
    assert cb.load_ms() > 0
    x, tgt, avail = C.queries(corpus.query, [], "cuda")
    out = cb.counts(x, tgt, avail, stats=True).cpu().numpy()
    ref = _reference(corpus, LEVELS, level_shards)
    top_tok = cb.top_tok.cpu().numpy().view(np.uint16)
    top_cnt = cb.top_cnt.cpu().numpy().view(np.uint32)
    for li, k in enumerate(LEVELS):
        o = ref[k]
        assert np.array_equal(out[0, li].view(np.uint32), o["tot"]), f"tot k={k}"
        assert np.array_equal(out[1, li].astype(np.uint16), o["dist"]), f"dist k={k}"
        assert np.array_equal(out[2, li].view(np.uint32), o["cnt"]), f"cnt k={k}"
        assert np.array_equal(top_tok[li], o["top_tok"][:, :4]), f"top_tok k={k}"
        assert np.array_equal(top_cnt[li], o["top_cnt"][:, :4]), f"top_cnt k={k}"
        assert cb.info[k]["hits"] == o["events"], f"hits k={k}"
    if mode in ("part", "list"):
        # a warm build (sizes learnt, no hit statistics): dense levels' query tables at their sparser load, the last
        # level's list scan without a bitmap, the device-listed query positions; the same outputs
        again = cb.counts(x, tgt, avail).cpu().numpy()
        assert np.array_equal(again, out)
        assert np.array_equal(cb.top_tok.cpu().numpy().view(np.uint16), top_tok)
        assert np.array_equal(cb.top_cnt.cpu().numpy().view(np.uint32), top_cnt)
    if mode == "regroup":
        assert cb.info[2]["pbits"] >= 3, cb.info[2]
    if mode == "regroup32":
        assert cb.engine.min_pbits.get(2, 0) > 11, cb.engine.min_pbits
    if mode == "wide":
        assert 2 in cb.engine.wide, cb.engine.wide
    if mode in ("part", "escape32", "regroup32"):
        assert not cb.engine.wide, cb.engine.wide
    assert (ref[2]["tot"] > 0).sum() > 1000 and (ref[20]["tot"] > 0).sum() > 10
    # the record's rows from ROW_LEVELS (ng_record_rows), and a batch of them (ng_batch_rows)
    tot_rows = np.stack([ref[k]["tot"] for k in C.ROW_LEVELS])
    cells, entries = O.record_rows(tot_rows, np.stack([ref[k]["top_tok"] for k in C.ROW_LEVELS]),
                                   np.stack([ref[k]["top_cnt"] for k in C.ROW_LEVELS]))
    assert np.array_equal(cb.row_cells.cpu().numpy(), cells)
    assert np.array_equal(cb.row_entries.cpu().numpy(), entries)
    n = 500
    cap = int((entries[1000 : 1000 + n] != 0).sum()) + 7
    assert np.array_equal(cb.batch_rows(1000, n, cap).cpu().numpy(), O.batch_rows(cells, entries, 1000, n, cap))
    with pytest.raises(AssertionError):
        cb.batch_rows(1000, n, cap - 8)


def test_warm_build_lists_query_positions_on_the_device(corpus, monkeypatch):
    """A build after the first lists each level's query positions on the device (no host read), in room sized from
    the last build's counts: after a build over a short query stream, the full stream's lists outrun that room, so
    the build runs once more with room for what it found; both builds match the oracle (the levels after an
    overflowed list, counted from a cut list, are not taken)."""
    cb = C.CountBuild(corpus.shards(), levels=LEVELS, level_shards={}, topk=4)
    cb.start_load(1)
    short = corpus.query[:20_001]
    xs, ts, avs = C.queries(short, [], "cuda")
    first = cb.counts(xs, ts, avs).cpu().numpy()
    seen_short = dict(cb.engine.seen_of)
    runs = []
    build = levels_mod.LevelBuild.build

    def counted(self, *a, **kw):
        runs.append(1)
        return build(self, *a, **kw)

    monkeypatch.setattr(levels_mod.LevelBuild, "build", counted)
    x, tgt, avail = C.queries(corpus.query, [], "cuda")
    out = cb.counts(x, tgt, avail).cpu().numpy()
    assert len(runs) >= 2, runs  # the device lists outran their room at least once
    assert all(cb.engine.seen_of[k] > seen_short[k] for k in seen_short)
    ref_short = _reference_for(short, corpus, LEVELS)
    ref = _reference(corpus, LEVELS, {})
    for li, k in enumerate(LEVELS):
        assert np.array_equal(first[0, li].view(np.uint32), ref_short[k]["tot"]), f"short tot k={k}"
        assert np.array_equal(first[2, li].view(np.uint32), ref_short[k]["cnt"]), f"short cnt k={k}"
        assert np.array_equal(out[0, li].view(np.uint32), ref[k]["tot"]), f"tot k={k}"
        assert np.array_equal(out[1, li].astype(np.uint16), ref[k]["dist"]), f"dist k={k}"
        assert np.array_equal(out[2, li].view(np.uint32), ref[k]["cnt"]), f"cnt k={k}"


def _reference_for(query, corpus, levels):
    x, tgt = query[:-1], query[1:]
    avail = O.segments(x)
    return {k: O.query_counts(corpus.train, corpus.bounds, x, tgt, avail, k, cnt_top=1 << 30, ntop=8) for k in levels}


def test_device_queries_match_host_queries(corpus):
    q = torch.from_numpy(corpus.query.view(np.int16)).cuda()
    a = C.device_queries(q)
    b = C.queries(corpus.query, [], "cuda")
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_fit_blocks_start_segments(corpus):
    blocks = [corpus.query[:300], corpus.query[300:700]]
    x, tgt, avail = C.queries(corpus.query[:1001], blocks, "cuda")
    av = avail.cpu().numpy()
    assert av[1000] == 1 and av[1000 + 299] == 1
    xs = np.concatenate([corpus.query[:1000], blocks[0][:-1], blocks[1][:-1]])
    assert np.array_equal(av, data.segments(xs, breaks=[1000, 1299]))


@pytest.mark.parametrize("margin", [1.2, 0.5])
def test_context_hints_from_an_earlier_build(corpus, monkeypatch, margin):
    """A build sizes its query indexes from the last build's context counts without reading them back before its
    scans: far fewer contexts than expected (the tables stand), then far more (inserts find no slot, so the build is
    done once more with every index's counters read: `redo` counts those builds); every build matches the oracle. A
    margin below 1 (every table fuller than its aimed load) still builds each index at most twice."""
    from ngram_amd import qindex as Q

    monkeypatch.setattr(Q, "EXPECT_MARGIN", margin)
    redo = []
    build = levels_mod.LevelBuild.build

    def counted(self, *a, **kw):
        redo.append(kw.get("_defer", True) is False)
        return build(self, *a, **kw)

    monkeypatch.setattr(levels_mod.LevelBuild, "build", counted)
    cb = C.CountBuild(corpus.shards(), levels=LEVELS, level_shards={}, topk=4)
    cb.start_load(1)
    full = corpus.query
    for j, q in enumerate((full, full[:3001], full)):
        redo.clear()
        x, tgt, avail = C.queries(q, [], "cuda")
        out = cb.counts(x, tgt, avail).cpu().numpy()
        assert any(redo) == (j == 2), (j, redo)
        xs, ts = q[:-1], q[1:]
        av = O.segments(xs)
        for li, k in enumerate(LEVELS):
            o = O.query_counts(corpus.train, corpus.bounds, xs, ts, av, k, cnt_top=1 << 30, ntop=4)
            assert np.array_equal(out[0, li].view(np.uint32), o["tot"]), (len(q), k)
            assert np.array_equal(out[2, li].view(np.uint32), o["cnt"]), (len(q), k)


@pytest.mark.parametrize("avail,closed", [([0, 1, 2, 3, 0, 1, 2], 1), ([1, 1, 1], 1), ([], 1), ([0, 1, 3], 0),
                                           ([2, 3], 0), ([0, 0, 5], 0), ([4, 5, 6, 1, 2], 0), ([1, 2, -3, 1], 1)])
def test_avail_closed_flag_by_hand(avail, closed):
    """ng_avail_closed: 1 iff avail[i] <= max(avail[i - 1], 0) + 1 wherever avail[i] > 1 (avail[-1] read as 0)."""
    from ngram_amd.lib import Lib

    a = torch.tensor(avail, dtype=torch.int32, device="cuda")
    flag = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    Lib()("ng_avail_closed", a, a.numel(), flag)
    assert int(flag.item()) == closed


def test_counts_with_holes_in_avail(corpus):
    """Query positions left unanswered (avail 0) break the prefix closure of the query contexts: the flag reads 0,
    the scans gate by the previous level's hit alone, and the build still matches the oracle run on the same avail;
    the same build with segment-shaped avail (the prefix rule on) matches it too."""
    from ngram_amd.lib import Lib

    x, tgt, avail = C.queries(corpus.query, [], "cuda")
    holes = avail.clone()
    holes[1000::997] = 0
    cb = C.CountBuild(corpus.shards(), levels=LEVELS, level_shards={}, topk=4)
    cb.start_load(1)
    xs, ts = corpus.query[:-1], corpus.query[1:]
    for av, closed in ((holes, 0), (avail, 1)):
        flag = torch.empty(1, dtype=torch.int32, device="cuda")
        Lib()("ng_avail_closed", av, av.numel(), flag)
        assert int(flag.item()) == closed
        out = cb.counts(x, tgt, av).cpu().numpy()
        a = av.cpu().numpy()
        for li, k in enumerate(LEVELS):
            o = O.query_counts(corpus.train, corpus.bounds, xs, ts, a, k, cnt_top=1 << 30, ntop=4)
            assert np.array_equal(out[0, li].view(np.uint32), o["tot"]), (closed, k)
            assert np.array_equal(out[1, li].astype(np.uint16), o["dist"]), (closed, k)
            assert np.array_equal(out[2, li].view(np.uint32), o["cnt"]), (closed, k)
            if closed == 0 and k == 3:
                assert (o["tot"][1001::997] > 0).any(), "a position after a hole has an occurring context"


def test_counts_from_device_tokens(corpus):
    """CountBuild.from_device (the shards already laid out in GPU memory, as the benchmark builds): every level's scan
    is one launch over all the shards, the first level included; tot / dist / cnt and the top-4 match the oracle, in
    a first build and in a second that uses the first one's densities and sizes."""
    tok, sizes, starts, L = data.device_tokens(corpus.shards())
    cb = C.CountBuild.from_device(tok, sizes, starts, levels=LEVELS, level_shards={}, topk=4)
    x, tgt, avail = C.queries(corpus.query, [], "cuda")
    ref = _reference(corpus, LEVELS, {})
    for stats in (True, False):
        out = cb.counts(x, tgt, avail, stats=stats).cpu().numpy()
        top_tok = cb.top_tok.cpu().numpy().view(np.uint16)
        top_cnt = cb.top_cnt.cpu().numpy().view(np.uint32)
        for li, k in enumerate(LEVELS):
            o = ref[k]
            assert np.array_equal(out[0, li].view(np.uint32), o["tot"]), (stats, k)
            assert np.array_equal(out[1, li].astype(np.uint16), o["dist"]), (stats, k)
            assert np.array_equal(out[2, li].view(np.uint32), o["cnt"]), (stats, k)
            assert np.array_equal(top_tok[li], o["top_tok"][:, :4]), (stats, k)
            assert np.array_equal(top_cnt[li], o["top_cnt"][:, :4]), (stats, k)


@pytest.mark.parametrize("packed", [False, True])
def test_emit_region_overflow_raises(corpus, monkeypatch, packed):
    """A scan whose per-block regions are too small for its hits flags it (the kernel keeps the hits it has room for
    and writes nothing past its region): the count raises before it reads a region, whether it reads the scan's flags
    with the event total of the regions' digit histograms or (packed: no histograms, the regions packed) on their
    own."""
    cb = C.CountBuild(corpus.shards(), levels=(2, 3), level_shards={}, topk=4)
    cb.start_load(1)
    x, tgt, avail = C.queries(corpus.query, [], "cuda")
    if packed:
        cb.counts(x, tgt, avail)  # a first build: its event counts let the next one go without digit histograms
        monkeypatch.setattr(P, "SEG_MIN_EVENTS", 1 << 40)
    monkeypatch.setattr(levels_mod, "emit_region", lambda L, G: 64)
    with pytest.raises(RuntimeError, match="emit region overflowed"):
        cb.counts(x, tgt, avail)


def test_event_total_of_2_32_or_more_raises():
    """count_events refuses a scan whose digit histograms sum to 2^32 events or more (the region scatter's offsets
    are u32): the scan's total is summed in 64 bits, so 2^32 + 5 does not wrap to 5 and the check fires before any
    region is read."""
    from ngram_amd.lib import Lib

    lib = Lib()
    nseg = 4
    regions = torch.zeros(nseg * 8, dtype=torch.int64, device="cuda")
    ev_count = torch.zeros(nseg, dtype=torch.int32, device="cuda")
    dhist = torch.zeros(256 * nseg, dtype=torch.int32, device="cuda")
    dhist[[3, 300, 600, 1000]] = 1 << 30
    dhist[7] = 5
    flags = torch.zeros(2, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="4294967301 events"):
        P.count_events(lib, lib, None, 0, 1000, 1.0, None, seg=(regions, 8, ev_count, dhist, nseg, flags))
