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
