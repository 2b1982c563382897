"""GPU: OnlineRows (exact_match's OnlineRows surface on libngram_amd.so, the step rule) against the oracle's
restatement of online.rs (pinned by brute force on tiny streams): advance step by step, hints / counts over a step
range, and a stream of several parts with interleaved steps."""

import numpy as np
import pytest

import oracle as O
from ngram_amd import data
from ngram_amd.online import OnlineRows

pytestmark = pytest.mark.gpu

LEVELS = [2, 3, 4, 5, 6]
BUCKETS = [2, 3, 4, 5, 6, 10, 20]


@pytest.fixture(scope="module")
def stream():
    zipf, plan, spans = data.c4_stream(steps=12, step_tokens=4096)
    return data.realize(plan, zipf), spans


def _empty(n, e, nc):
    return (np.zeros(n, np.int16), np.zeros((n, e), np.uint16), np.zeros((n, e), np.uint16),
            np.zeros((n, nc), np.uint32), np.zeros((n, nc), np.uint16), np.zeros((n, nc), np.uint32))


@pytest.mark.parametrize("entries", [8, 3])
def test_advance_step_by_step(stream, entries):
    tok, spans = stream
    n = len(tok)
    bounds = [0, n]
    tau, tau_in = O.spans_tau(n, bounds, spans)
    want = O.online(tok, bounds, tau, tau_in, LEVELS, BUCKETS, entries, LEVELS, 0, len(spans))
    rows = OnlineRows(tok, bounds, spans, 4, [])
    got = _empty(n, entries, len(LEVELS))
    hinted = 0
    for s in range(len(spans)):
        hinted += rows.advance(s + 1, LEVELS, BUCKETS, entries, LEVELS, *got)
    assert rows.done == len(spans) and len(rows) == n
    for g, w, name in zip(got, want, ("cell", "next", "weights", "tot", "dist", "cnt")):
        assert np.array_equal(g, w), name
    assert hinted == want[-1] and hinted > n // 10


def test_hints_and_counts_ranges(stream):
    tok, spans = stream
    n = len(tok)
    bounds = [0, n]
    tau, tau_in = O.spans_tau(n, bounds, spans)
    rows = OnlineRows(tok, bounds, spans, 4, [])
    cell, nxt, w = np.zeros(n, np.int16), np.zeros((n, 8), np.uint16), np.zeros((n, 8), np.uint16)
    h = rows.hints([3, 5], BUCKETS, 8, 4, 9, cell, nxt, w)
    want = O.online(tok, bounds, tau, tau_in, [3, 5], BUCKETS, 8, [], 4, 9)
    assert h == want[-1]
    for g, x in zip((cell, nxt, w), want[:3]):
        assert np.array_equal(g, x)
    tot, dist, cnt = np.zeros((n, 2), np.uint32), np.zeros((n, 2), np.uint16), np.zeros((n, 2), np.uint32)
    rows.counts([2, 4], 2, 7, tot, dist, cnt)
    want = O.online(tok, bounds, tau, tau_in, [], [1], 1, [2, 4], 2, 7)
    for g, x in zip((tot, dist, cnt), want[3:6]):
        assert np.array_equal(g, x)


def test_parts_and_interleaved_steps():
    rng = np.random.default_rng(7)
    shards = [data.make_corpus("c1", train_tokens=20_000, query_tokens=2, shard_tokens=20_000).train[i * 5000:(i + 1) * 5000]
              for i in range(3)]
    tok = np.concatenate(shards)
    bounds = [0, 5000, 10000, 15000]
    spans = []
    for j in range(3):  # each part consumed in 5 chunks; the parts' steps interleave
        cuts = np.linspace(bounds[j], bounds[j + 1] - 1, 6).astype(int)
        for s in range(5):
            spans.append((cuts[s], cuts[s + 1], s + int(rng.integers(0, 2))))
    spans = np.array(spans, np.int64)
    n = len(tok)
    tau, tau_in = O.spans_tau(n, bounds, spans)
    steps = int(spans[:, 2].max()) + 1
    want = O.online(tok, bounds, tau, tau_in, [1, 2, 4], [1, 2, 3, 4], 4, [1, 3], 0, steps)
    rows = OnlineRows(tok, bounds, spans, 4, [])
    got = _empty(n, 4, 2)
    rows.advance(2, [1, 2, 4], [1, 2, 3, 4], 4, [1, 3], *got)
    rows.advance(steps, [1, 2, 4], [1, 2, 3, 4], 4, [1, 3], *got)
    for g, w, name in zip(got, want, ("cell", "next", "weights", "tot", "dist", "cnt")):
        assert np.array_equal(g, w), name


@pytest.mark.parametrize("seed", range(4))
def test_segment_rule_matches_brute_force(seed):
    """rule="segment" (online.rs:14-17: every position answered from its segment's start) for hints and counts on
    small random streams of several parts, against the rule's brute force (itself pinned by hand)."""
    rng = np.random.default_rng(40 + seed)
    n = int(rng.integers(150, 260))
    tok = rng.integers(0, 4, size=n).astype(np.uint16)
    tok[rng.random(n) < 0.06] = O.BOS
    cuts = sorted(rng.choice(np.arange(20, n - 20), size=int(rng.integers(0, 3)), replace=False).tolist())
    bounds = [0] + cuts + [n]
    rows = OnlineRows(tok, bounds, np.zeros((0, 3), np.int64))  # the rule ignores the spans
    levels, buckets, E, cl = [1, 2, 3], [1, 2, 3, 4], 3, [1, 2, 4]
    want = O.brute_segment(tok, bounds, levels, buckets, E, cl)
    cell, nxt, w = np.zeros(n, np.int16), np.zeros((n, E), np.uint16), np.zeros((n, E), np.uint16)
    hinted = rows.hints(levels, buckets, E, 0, 0, cell, nxt, w, rule="segment")
    tot, dist, cnt = np.zeros((n, 3), np.uint32), np.zeros((n, 3), np.uint16), np.zeros((n, 3), np.uint32)
    rows.counts(cl, 0, 0, tot, dist, cnt, rule="segment")
    for g, x, name in zip((cell, nxt, w, tot, dist, cnt), want, ("cell", "next", "weights", "tot", "dist", "cnt")):
        assert np.array_equal(g, x), name
    assert hinted == want[-1] and hinted > 0


def test_segment_rule_on_parts_of_a_real_stream():
    """rule="segment" over three parts of the c1 generator's stream (15K tokens, a few dozen segments) against the
    oracle's online restatement fed the segment indices as the steps."""
    shards = [data.make_corpus("c1", train_tokens=20_000, query_tokens=2, shard_tokens=20_000).train[i * 5000:(i + 1) * 5000]
              for i in range(3)]
    tok = np.concatenate(shards)
    n, bounds = len(tok), [0, 5000, 10000, 15000]
    starts = np.zeros(n, bool)
    starts[bounds[:-1]] = True
    starts |= tok == O.BOS
    seg = (np.cumsum(starts) - 1).astype(np.uint32)
    want = O.online(tok, bounds, seg, seg, [1, 2, 4], [1, 2, 3, 4], 4, [1, 3], 0, int(seg[-1]) + 1)
    rows = OnlineRows(tok, bounds, np.zeros((0, 3), np.int64))
    cell, nxt, w = np.zeros(n, np.int16), np.zeros((n, 4), np.uint16), np.zeros((n, 4), np.uint16)
    assert rows.hints([1, 2, 4], [1, 2, 3, 4], 4, 0, 0, cell, nxt, w, rule="segment") == want[-1]
    tot, dist, cnt = np.zeros((n, 2), np.uint32), np.zeros((n, 2), np.uint16), np.zeros((n, 2), np.uint32)
    rows.counts([1, 3], 0, 0, tot, dist, cnt, rule="segment")
    for g, x, name in zip((cell, nxt, w, tot, dist, cnt), want, ("cell", "next", "weights", "tot", "dist", "cnt")):
        assert np.array_equal(g, x), name
    assert seg[-1] > 10


def test_loader_plan_rows():
    """A training run planned by llm.c's sequential loader (2 ranks, B*T = 256, 2 micro-steps): the stream's parts and
    spans from the plan, OnlineRows advanced over its steps against the oracle, and each rank's rows gathered in
    training order."""
    from ngram_amd.online import loader_plan, plan_rows, plan_spans, plan_stream

    c = data.make_corpus("c1", train_tokens=12_000, query_tokens=2, shard_tokens=12_000).train
    ntok = [4000, 5000, 3000]
    shards = [c[:4000], c[4000:9000], c[9000:12000]]
    plan = loader_plan(ntok, 2, 256, 2, 9)  # 18 micro-batches a rank: 7 in shard 0, 9 in shard 1, 2 in shard 2
    sizes = plan_stream(ntok, plan, 256)
    tok = np.concatenate([shards[j][: sizes[j]] for j in range(len(sizes))])
    bounds = np.concatenate([[0], np.cumsum(sizes)]).tolist()
    spans = plan_spans(plan, sizes, 256)
    n = len(tok)
    tau, tau_in = O.spans_tau(n, bounds, spans)
    want = O.online(tok, bounds, tau, tau_in, [1, 2, 3], [1, 2, 3], 4, [2, 3], 0, 9)
    rows = OnlineRows(tok, bounds, spans)
    got = _empty(n, 4, 2)
    rows.advance(9, [1, 2, 3], [1, 2, 3], 4, [2, 3], *got)
    for g, w, name in zip(got, want, ("cell", "next", "weights", "tot", "dist", "cnt")):
        assert np.array_equal(g, w), name
    for r in range(2):
        at = plan_rows(plan, sizes, 256, 2, r)
        assert len(at) == 9 * 2 * 256 and (at >= 0).all() and len(np.unique(at)) == len(at)
        assert np.array_equal(got[0][at], want[0][at]) and (got[0][at] != 0).mean() > 0.3
    assert len(sizes) == 3


def test_errors(stream):
    tok, spans = stream
    n = len(tok)
    with pytest.raises(ValueError):
        OnlineRows(tok, [0, n - 1], spans)
    with pytest.raises(ValueError):
        OnlineRows(tok, [0, n], np.array([[5, 3, 0]]))
    rows = OnlineRows(tok, [0, n], spans)
    rows.advance(1, LEVELS, BUCKETS, 8, LEVELS)
    with pytest.raises(ValueError):
        rows.advance(2, [2, 3], BUCKETS, 8, LEVELS)  # the configuration is fixed
    with pytest.raises(ValueError):
        rows.hints([7], BUCKETS, 8, 0, 1, np.zeros(n, np.int16), np.zeros((n, 8), np.uint16),
                   np.zeros((n, 8), np.uint16))


class _PerLevelRows(OnlineRows):
    """OnlineRows whose steps use the single-level entry points: ng_online_insert per level (pairs counted per
    occurrence), ng_online_top without add_counts, ng_online_query per level. The same outputs are expected."""

    def _step(self, st, s, outs, queries=True):
        from ngram_amd.lib import i32, u64

        lib = self.lib
        levels, buckets, entries, count_levels = outs["cfg"]
        m = 0
        for t, (k, lv) in enumerate(st["levels"].items()):
            a, b = self._range(lv["alpha"], s, s + 1)
            if b == a:
                continue
            lib("ng_online_insert", self.tok, lv["occ"][a:b], b - a, i32(k), lv["ck"], u64(lv["ccap"]), lv["pt"],
                u64(lv["pcap"]), None, i32(0), st["ev"][m:], lv["flags"], u64(t << st["tshift"]))
            m += b - a
        if m:
            lib.cub("sort_pairs", st["ev"], st["ev_sorted"], None, None, m, i32(0), i32(st["tshift"] + st["tag_bits"]))
            lib.cub("reduce_by_key", st["ev_sorted"], st["uk"], None, st["agg"], st["nruns"], m)
            lib("ng_online_top", st["uk"], st["nruns"], m, st["agg"], st["top_desc"], i32(len(st["levels"])),
                i32(st["tshift"]), st["score"], i32(st["E"]), i32(0))
        qa, qb = self._range(st["q_step"], s, s + 1)
        if qb == qa or not queries:
            return
        qpos = st["q_pos"][qa:qb]
        for ci, k in enumerate(count_levels):
            lv = st["levels"][k]
            lib("ng_online_query", self.tok, self.avail, self.has_next, qpos, qb - qa, i32(k), lv["ck"],
                u64(lv["ccap"]), lv["pt"], u64(lv["pcap"]), lv["rec"], i32(lv["rw"]),
                st["qslot"][k] if k in levels else None, outs["tot"], outs["dist"], outs["cnt"], i32(len(count_levels)),
                i32(ci))
        for k in levels:
            if k not in count_levels:
                lv = st["levels"][k]
                lib("ng_online_query", self.tok, self.avail, self.has_next, qpos, qb - qa, i32(k), lv["ck"],
                    u64(lv["ccap"]), lv["pt"], u64(lv["pcap"]), lv["rec"], i32(lv["rw"]), st["qslot"][k],
                    None, None, None, i32(1), i32(0))
        if levels:
            lib("ng_online_rows", qpos, qb - qa, i32(len(levels)), st["rows_desc"], i32(st["E"]), i32(outs["slots"]),
                outs["cell"], outs["next"], outs["weights"], outs["level"], st["hinted"])


@pytest.mark.parametrize("how", ["per_level", "chunks_of_3", "sorted"])
def test_step_entry_points_agree(stream, monkeypatch, how):
    """The single-level entry points (pairs counted per occurrence), the fused launches split in chunks of three
    levels, and the sorted merge (sort_pairs + reduce_by_key + ng_online_top in place of ng_online_merge) give the
    oracle's rows, as the default path does (test_advance_step_by_step)."""
    from ngram_amd import online as on

    tok, spans = stream
    n = len(tok)
    bounds = [0, n]
    tau, tau_in = O.spans_tau(n, bounds, spans)
    count_levels = [2, 4, 6]
    want = O.online(tok, bounds, tau, tau_in, LEVELS, BUCKETS, 8, count_levels, 0, len(spans))
    if how == "per_level":
        rows = _PerLevelRows(tok, bounds, spans, 4, [])
        rows.merge = "sorted"  # its steps use the sorted merge's buffers
    elif how == "sorted":
        rows = OnlineRows(tok, bounds, spans, 4, [])
        rows.merge = "sorted"
    else:
        monkeypatch.setattr(on, "MAX_LAUNCH_LEVELS", 3)
        rows = OnlineRows(tok, bounds, spans, 4, [])
    got = _empty(n, 8, len(count_levels))
    hinted = rows.advance(len(spans), LEVELS, BUCKETS, 8, count_levels, *got)
    for g, w, name in zip(got, want, ("cell", "next", "weights", "tot", "dist", "cnt")):
        assert np.array_equal(g, w), name
    assert hinted == want[-1]


@pytest.mark.parametrize("merge", ["buckets", "sorted"])
def test_context_with_more_pairs_than_a_merge_round(merge):
    """A level-2 context followed by 6000 distinct tokens within one step: its bucket holds more distinct pairs than
    ng_online_merge's LDS round (4096), so the bucket is merged in rounds split by a pair hash, the context's pairs
    spread over them; the next steps touch half of those pairs again and add new ones. Rows and counts against the
    oracle, for both merges."""
    rng = np.random.default_rng(11)
    a, b = 7, 9
    seq = []
    for j in range(6000):
        seq += [a, b, 1000 + j]
    for j in range(3000, 9000):
        seq += [a, b, 1000 + j % 7000, int(rng.integers(0, 50))]
    seq += list(rng.integers(0, 300, 20000))
    tok = np.array(seq, np.uint16)
    n = len(tok)
    cuts = [0, 18000, 42000, n]
    spans = np.array([(cuts[s], cuts[s + 1], s) for s in range(3)], np.int64)
    bounds = [0, n]
    tau, tau_in = O.spans_tau(n, bounds, spans)
    want = O.online(tok, bounds, tau, tau_in, LEVELS, BUCKETS, 8, LEVELS, 0, len(spans))
    rows = OnlineRows(tok, bounds, spans, 4, [])
    rows.merge = merge
    got = _empty(n, 8, len(LEVELS))
    hinted = rows.advance(len(spans), LEVELS, BUCKETS, 8, LEVELS, *got)
    if merge == "buckets":
        assert rows.state["merge_temp"] is not None
    for g, w, name in zip(got, want, ("cell", "next", "weights", "tot", "dist", "cnt")):
        assert np.array_equal(g, w), name
    assert hinted == want[-1]
    assert int(got[3][:, 0].max()) >= 6000  # the context's total reached the step's 6000 occurrences


def test_many_count_levels(stream):
    """Eight levels in one step's merge (three tag bits in the packed words) against the oracle's counts; nine levels
    (more than ng_online_merge takes: the sorted merge runs) against those and, for the level past the oracle's
    eight-token limit, the same level counted alone by the bucketed merge."""
    tok, spans = stream
    n = len(tok)
    bounds = [0, n]
    tau, tau_in = O.spans_tau(n, bounds, spans)
    eight = [1, 2, 3, 4, 5, 6, 7, 8]
    want = O.online(tok, bounds, tau, tau_in, [], [1], 1, eight, 0, len(spans))

    def counts(levels):
        nc = len(levels)
        out = np.zeros((n, nc), np.uint32), np.zeros((n, nc), np.uint16), np.zeros((n, nc), np.uint32)
        OnlineRows(tok, bounds, spans, 4, []).counts(levels, 0, len(spans), *out)
        return out

    got8, got9, alone = counts(eight), counts(eight + [10]), counts([10])
    for j, name in enumerate(("tot", "dist", "cnt")):
        assert np.array_equal(got8[j], want[3 + j]), name
        assert np.array_equal(got9[j][:, :8], want[3 + j]), name
        assert np.array_equal(got9[j][:, 8:], alone[j]), name
    assert int(got8[0].max()) > 0 and int(alone[0].max()) > 0
