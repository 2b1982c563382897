"""CPU oracle of the n-gram hint path: TEST INFRASTRUCTURE ONLY (the checker; and, timed, bench.py's CPU baseline).
Nothing in the product imports this module.

* `query_counts` / `table_counts` / `longest_match`: ctypes over liboracle.so (oracle.cpp: the C++ restatement of
  exact_match/src/kgram.rs count_with + scan + Contexts and of exact_match/src/count_table.rs build_level + runs +
  query_counts).
* `brute_counts` / `brute_longest`: pure-Python brute force (collections.Counter over every (context tuple, next) of
  every shard) straight from the definitions of kgram.rs:7-9 -- for tiny inputs, to pin the C++ restatement.
* numpy restatements of the reference's post-processing:
  - `deepest_rows`: src/retrieval_blog_post/val_hints.py deepest (:277-311) + old_records.py _val_rows_range
    (:102-124) + _weights (:70-73), packed as old_records/gpu_val_stats.cu variant_rows (:646-694): int32 [N, 9].
  - `features`: record_367_gpu_counts/track_1_short/counts/mix.py features (:22-31), float32.
  - `record_rows`: record_367_gpu_counts/track_1_short/counts/build.py counts() rows (:341-387) and batch_rows
    (:390-403).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from collections import Counter, defaultdict
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle.so"
BOS = 50256
TOP = 1024
LEVELS = (2, 3, 4, 5, 6, 10, 20)
ALL_LEVELS = (2, 3, 4, 5, 6, 8, 10, 12, 16, 20)
COUNT_EDGES = (2, 3, 5, 9, 17, 33)
PURITY_EDGES = (0.3, 0.5, 0.7, 0.85, 0.95)
WEIGHT_ONE = 65535
NB = 25

_lib = None


def build() -> Path:
    """Compile liboracle.so (make in this directory)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        so = ctypes.CDLL(str(LIB))
        P = ctypes.c_void_p
        so.oracle_query_counts.restype = ctypes.c_int64
        so.oracle_query_counts.argtypes = [P, P, ctypes.c_int, P, P, P, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int, P, P, P, P, P, P, P, ctypes.c_int]
        so.oracle_table_counts.restype = ctypes.c_int64
        so.oracle_table_counts.argtypes = [P, P, ctypes.c_int, P, P, P, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int, P, P, P, P, P, P, P, ctypes.c_int]
        so.oracle_online.restype = ctypes.c_int64
        so.oracle_online.argtypes = [P, ctypes.c_int64, P, ctypes.c_int, P, P, P, ctypes.c_int, P, ctypes.c_int,
                                     ctypes.c_int, P, ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32, P, P, P, P, P, P,
                                     ctypes.c_int]
        so.oracle_longest_match.restype = ctypes.c_int
        so.oracle_longest_match.argtypes = [P, P, ctypes.c_int, P, P, ctypes.c_int64, ctypes.c_int, P, P, P,
                                            ctypes.c_int]
        _lib = so
    return _lib


def _p(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def threads() -> int:
    return max(1, len(os.sched_getaffinity(0)))


def segments(x: np.ndarray, breaks=()) -> np.ndarray:
    """kgram.rs segments (:224-234) with extra segment starts (kgram_query_counts' breaks, :145-152)."""
    n = len(x)
    avail = np.zeros(n, np.int32)
    start = 0
    bset = set(breaks)
    xs = np.asarray(x)
    starts = np.flatnonzero(xs == BOS)
    mark = np.zeros(n, bool)
    mark[starts] = True
    for b in bset:
        mark[b] = True
    if n:
        mark[0] = True
    idx = np.arange(n)
    seg = np.maximum.accumulate(np.where(mark, idx, 0))
    avail[:] = idx - seg + 1
    del start
    return avail


class Outputs(dict):
    """Per-position outputs of one level: tot u32, dist u16, cnt u32, top_tok u16 [N, ntop], top_cnt u32 [N, ntop]."""


def _alloc(n: int, ntop: int) -> Outputs:
    return Outputs(tot=np.zeros(n, np.uint32), dist=np.zeros(n, np.uint16), cnt=np.zeros(n, np.uint32),
                   top_tok=np.zeros((n, max(ntop, 1)), np.uint16), top_cnt=np.zeros((n, max(ntop, 1)), np.uint32))


def query_counts(train: np.ndarray, bounds: np.ndarray, x: np.ndarray, tgt: np.ndarray, avail: np.ndarray, k: int,
                 cnt_top: int = TOP, ntop: int = 8, nthreads: int | None = None, hits: bool = False,
                 gate: np.ndarray | None = None) -> Outputs:
    """Query-filtered counts of level k (kgram.rs restatement). `train` is the shards concatenated, shard s being
    train[bounds[s]:bounds[s+1]]. `hits`: also the corpus positions whose k-context matched (uint8 per position).
    `gate` (uint8 per corpus position, e.g. the previous level's hits): only its set positions are examined -- exact
    for the levels above the gate's, since a k-context occurs only where its (k-1)-suffix does (kgram.rs:12-15)."""
    train = np.ascontiguousarray(train, np.uint16)
    bounds = np.ascontiguousarray(bounds, np.int64)
    x = np.ascontiguousarray(x, np.uint16)
    tgt = np.ascontiguousarray(tgt, np.uint16)
    avail = np.ascontiguousarray(avail, np.int32)
    if gate is not None:
        gate = np.ascontiguousarray(gate, np.uint8)
        if len(gate) != len(train):
            raise ValueError("gate needs one byte per corpus position")
    out = _alloc(len(x), ntop)
    hb = np.zeros(len(train), np.uint8) if hits else None
    events = lib().oracle_query_counts(_p(train), _p(bounds), len(bounds) - 1, _p(x), _p(tgt), _p(avail), len(x), k,
                                       cnt_top, max(ntop, 1), _p(out["tot"]), _p(out["dist"]), _p(out["cnt"]),
                                       _p(out["top_tok"]), _p(out["top_cnt"]), _p(hb), _p(gate), nthreads or threads())
    if events < 0:
        raise ValueError("oracle_query_counts: bad arguments")
    out["events"] = int(events)
    if hits:
        out["hits"] = hb
    return out


def table_counts(train: np.ndarray, bounds: np.ndarray, x: np.ndarray, tgt: np.ndarray, avail: np.ndarray, k: int,
                 cnt_top: int = TOP, ntop: int = 8, nthreads: int | None = None) -> Outputs:
    """Corpus-wide counts of level k <= 8 (count_table.rs restatement), queried at the positions."""
    train = np.ascontiguousarray(train, np.uint16)
    bounds = np.ascontiguousarray(bounds, np.int64)
    x = np.ascontiguousarray(x, np.uint16)
    tgt = np.ascontiguousarray(tgt, np.uint16)
    avail = np.ascontiguousarray(avail, np.int32)
    out = _alloc(len(x), ntop)
    nc = np.zeros(1, np.int64)
    npairs = np.zeros(1, np.int64)
    events = lib().oracle_table_counts(_p(train), _p(bounds), len(bounds) - 1, _p(x), _p(tgt), _p(avail), len(x), k,
                                       cnt_top, max(ntop, 1), _p(out["tot"]), _p(out["dist"]), _p(out["cnt"]),
                                       _p(out["top_tok"]), _p(out["top_cnt"]), _p(nc), _p(npairs),
                                       nthreads or threads())
    if events < 0:
        raise ValueError("oracle_table_counts: bad arguments")
    out["events"], out["contexts"], out["pairs"] = int(events), int(nc[0]), int(npairs[0])
    return out


def longest_match(train: np.ndarray, bounds: np.ndarray, x: np.ndarray, avail: np.ndarray, cap: int,
                  nthreads: int | None = None) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Per position: the longest valid k <= cap whose k-context occurred, its top next token and that count."""
    train = np.ascontiguousarray(train, np.uint16)
    bounds = np.ascontiguousarray(bounds, np.int64)
    x = np.ascontiguousarray(x, np.uint16)
    avail = np.ascontiguousarray(avail, np.int32)
    n = len(x)
    length = np.zeros(n, np.uint32)
    nxt = np.zeros(n, np.uint16)
    cnt = np.zeros(n, np.uint32)
    rc = lib().oracle_longest_match(_p(train), _p(bounds), len(bounds) - 1, _p(x), _p(avail), n, cap, _p(length),
                                    _p(nxt), _p(cnt), nthreads or threads())
    if rc:
        raise ValueError("oracle_longest_match: bad arguments")
    return length, nxt, cnt


NONE = 0xFFFFFFFF


def spans_tau(n: int, bounds, spans) -> tuple[np.ndarray, np.ndarray]:
    """online.rs new (:137-158): tau (first step training a position as input or target) and tau_in (as input) from
    spans (lo, hi, step): inputs [lo, hi) of `step`, position hi its last target if within the part of hi - 1."""
    tau = np.full(n, NONE, np.uint32)
    tau_in = np.full(n, NONE, np.uint32)
    b = np.asarray(bounds, np.int64)
    for lo, hi, step in np.asarray(spans, np.int64).reshape(-1, 3):
        tau[lo:hi] = np.minimum(tau[lo:hi], step)
        tau_in[lo:hi] = np.minimum(tau_in[lo:hi], step)
        if hi > lo and hi < n:
            part = int(np.searchsorted(b, hi - 1, side="right"))
            if hi < b[part]:
                tau[hi] = min(tau[hi], step)
    return tau, tau_in


def online(tokens, bounds, tau, tau_in, levels, buckets, entries, count_levels, step_lo: int, step_hi: int,
           nthreads: int | None = None):
    """The step rule's hint rows and count rows (oracle_online): (cell int16 [n], next uint16 [n, entries], weights
    uint16 [n, entries], tot uint32 [n, nc], dist uint16 [n, nc], cnt uint32 [n, nc], queries hinted)."""
    tok = np.ascontiguousarray(tokens, np.uint16)
    n = len(tok)
    b = np.ascontiguousarray(bounds, np.int64)
    lv = np.ascontiguousarray(levels, np.int32)
    bk = np.ascontiguousarray(buckets, np.int32)
    cl = np.ascontiguousarray(count_levels, np.int32)
    cell = np.zeros(n, np.int16)
    nxt = np.zeros((n, entries), np.uint16)
    w = np.zeros((n, entries), np.uint16)
    tot = np.zeros((n, max(len(cl), 1)), np.uint32)
    dist = np.zeros((n, max(len(cl), 1)), np.uint16)
    cnt = np.zeros((n, max(len(cl), 1)), np.uint32)
    hinted = lib().oracle_online(_p(tok), n, _p(b), len(b) - 1, _p(np.ascontiguousarray(tau, np.uint32)),
                                 _p(np.ascontiguousarray(tau_in, np.uint32)), _p(lv), len(lv), _p(bk), len(bk), entries,
                                 _p(cl), len(cl), step_lo, step_hi, _p(cell), _p(nxt), _p(w), _p(tot), _p(dist),
                                 _p(cnt), nthreads or threads())
    if hinted < 0:
        raise ValueError("oracle_online: bad arguments")
    return cell, nxt, w, tot[:, : len(cl)], dist[:, : len(cl)], cnt[:, : len(cl)], int(hinted)


def brute_online(tokens, bounds, tau, tau_in, levels, buckets, entries, count_levels, step_lo, step_hi):
    """online.rs's definitions directly (tiny inputs), the step rule: per query (a position trained as an input in
    [step_lo, step_hi)) and level, every valid occurrence of its context with alpha <= the query's step counted from
    scratch."""
    tok = [int(t) for t in tokens]

    def alpha(h, k, part_lo, part_hi):
        ts = [int(tau[q]) for q in range(h - k + 1, h + 2)]
        return None if NONE in ts else 1 + max(ts)

    queries = [g for g in range(len(tok)) if tau_in[g] != NONE and step_lo <= tau_in[g] < step_hi]
    return _brute_rows(tok, bounds, levels, buckets, entries, count_levels, queries,
                       lambda h, g, k, seg, lo, hi: (a := alpha(h, k, lo, hi)) is not None and a <= tau_in[g])


def brute_segment(tokens, bounds, levels, buckets, entries, count_levels):
    """online.rs's rule "segment" directly (tiny inputs, online.rs:14-17): every position with a valid context is a
    query, and an occurrence (its k tokens and next token within one part) counts for it iff its next token lies
    before the query's segment start."""
    tok = [int(t) for t in tokens]
    return _brute_rows(tok, bounds, levels, buckets, entries, count_levels, list(range(len(tok))),
                       lambda h, g, k, seg, lo, hi: h + 1 < seg[g])


def brute_train_hints(tokens, bounds, levels, buckets, entries, slots):
    """train_hints.rs's rows directly (tiny inputs): every position's deepest `slots` levels with an occurrence counted
    under the rule "segment", deepest first: cell [n, slots], next / weights [n, slots, entries], level [n, slots]
    (the level's index in `buckets`, -1 for an empty slot)."""
    tok = [int(t) for t in tokens]
    return _brute_rows(tok, bounds, levels, buckets, entries, [], list(range(len(tok))),
                       lambda h, g, k, seg, lo, hi: h + 1 < seg[g], slots=slots)


def _brute_rows(tok, bounds, levels, buckets, entries, count_levels, queries, counts_for, slots=None):
    """Rows of `queries` from scratch: counts_for(h, g, k, seg, part_lo, part_hi) says whether the occurrence ending at
    h (valid within its part) counts for the query at g. With `slots`, hint rows in that many slots (deepest levels
    first) and their levels: (cell, next, weights, level)."""
    n = len(tok)
    part_lo, part_hi, seg = [0] * n, [0] * n, [0] * n
    for a, bnd in zip(bounds[:-1], bounds[1:]):
        s0 = a
        for g in range(a, bnd):
            if tok[g] == BOS:
                s0 = g
            part_lo[g], part_hi[g], seg[g] = a, bnd, s0
    nc = len(count_levels)
    tot = np.zeros((n, nc), np.uint32)
    dist = np.zeros((n, nc), np.uint16)
    cnt = np.zeros((n, nc), np.uint32)

    def table(g, k):
        c = tok[g - k + 1 : g + 1]
        found = Counter()
        for h in range(n):
            if h - k + 1 < part_lo[h] or h + 1 >= part_hi[h]:
                continue
            if counts_for(h, g, k, seg, part_lo, part_hi) and tok[h - k + 1 : h + 1] == c:
                found[tok[h + 1]] += 1
        return found

    S = slots or 1
    scell = np.zeros((n, S), np.int16)
    snxt = np.zeros((n, S, entries), np.uint16)
    sw = np.zeros((n, S, entries), np.uint16)
    slevel = np.full((n, S), -1, np.int8)
    hinted = 0
    for g in queries:
        for j, k in enumerate(count_levels):
            if g - seg[g] + 1 < k:
                continue
            f = table(g, k)
            if f:
                tot[g, j] = sum(f.values())
                dist[g, j] = min(len(f), 65535)
                cnt[g, j] = f[tok[g + 1]] if g + 1 < part_hi[g] else 0
        j = 0
        for k in sorted(levels, reverse=True):
            if j == S:
                break
            if g - seg[g] + 1 < k:
                continue
            f = table(g, k)
            if not f:
                continue
            ranked = sorted(f.items(), key=lambda tc: (-tc[1], tc[0]))[:entries]
            total = sum(f.values())
            li = list(buckets).index(k)
            cb = sum(e <= total for e in COUNT_EDGES)
            pb = sum(e <= ranked[0][1] / total for e in PURITY_EDGES)
            scell[g, j] = ((1 + li) * 7 + cb) * 6 + pb
            slevel[g, j] = li
            s = float(sum(c for _, c in ranked))
            for r, (t, c) in enumerate(ranked):
                snxt[g, j, r] = t
                sw[g, j, r] = int(np.round(c / s * WEIGHT_ONE))
            j += 1
        hinted += j > 0
    if slots is not None:
        return scell, snxt, sw, slevel
    return scell[:, 0], snxt[:, 0], sw[:, 0], tot, dist, cnt, hinted


# ---------------------------------------------------------------------------------------------------------------
# Brute force (tiny inputs)
# ---------------------------------------------------------------------------------------------------------------

def brute_table(shards: list[np.ndarray], k: int) -> dict[tuple, Counter]:
    """Every occurrence of every k-context: context tuple -> Counter of next tokens."""
    table: dict[tuple, Counter] = defaultdict(Counter)
    for s in shards:
        s = [int(t) for t in s]
        for p in range(k, len(s)):
            table[tuple(s[p - k : p])][s[p]] += 1
    return table


def brute_counts(shards: list[np.ndarray], x: np.ndarray, tgt: np.ndarray, avail: np.ndarray, k: int,
                 cnt_top: int = TOP, ntop: int = 8) -> Outputs:
    table = brute_table(shards, k)
    n = len(x)
    out = _alloc(n, ntop)
    for i in range(n):
        if avail[i] < k:
            continue
        c = table.get(tuple(int(t) for t in x[i + 1 - k : i + 1]))
        if not c:
            continue
        ranked = sorted(c.items(), key=lambda tc: (-tc[1], tc[0]))
        out["tot"][i] = sum(c.values())
        out["dist"][i] = min(len(c), 65535)
        for r, (t, m) in enumerate(ranked[:cnt_top]):
            if t == tgt[i]:
                out["cnt"][i] = m
                break
        for r, (t, m) in enumerate(ranked[:ntop]):
            out["top_tok"][i, r] = t
            out["top_cnt"][i, r] = m
    return out


def brute_longest(shards: list[np.ndarray], x: np.ndarray, avail: np.ndarray, cap: int):
    n = len(x)
    length = np.zeros(n, np.uint32)
    nxt = np.zeros(n, np.uint16)
    cnt = np.zeros(n, np.uint32)
    for k in range(1, cap + 1):
        table = brute_table(shards, k)
        for i in range(n):
            if avail[i] < k:
                continue
            c = table.get(tuple(int(t) for t in x[i + 1 - k : i + 1]))
            if c:
                t, m = sorted(c.items(), key=lambda tc: (-tc[1], tc[0]))[0]
                length[i], nxt[i], cnt[i] = k, t, m
    return length, nxt, cnt


# ---------------------------------------------------------------------------------------------------------------
# Post-processing restatements
# ---------------------------------------------------------------------------------------------------------------

def weights(counts: np.ndarray) -> np.ndarray:
    """old_records.py _weights (:70-73): counts [..., 8] as weights summing to 65535 (round half even, float64)."""
    total = counts.sum(-1, keepdims=True, dtype=np.float64)
    return np.round(counts / np.maximum(total, 1) * WEIGHT_ONE).astype(np.uint16)


def deepest_rows(per_level: dict[int, Outputs], variant: tuple[int, ...], buckets: tuple[int, ...] = LEVELS):
    """The variant's hint rows (val_hints.deepest + _val_rows + _weights): per position its deepest level of `variant`
    whose context occurred -> (cell int16 [N], tokens uint16 [N, 8], weights uint16 [N, 8])."""
    n = len(next(iter(per_level.values()))["tot"])
    level = np.full(n, -1, np.int64)
    total = np.zeros(n, np.uint64)
    top = np.zeros(n, np.uint64)
    tokens = np.zeros((n, 8), np.uint16)
    counts = np.zeros((n, 8), np.uint64)
    filled = np.zeros(n, bool)
    for k in reversed(variant):
        o = per_level[k]
        at = np.flatnonzero((o["tot"] > 0) & ~filled)
        level[at] = buckets.index(k)
        total[at] = o["tot"][at]
        top[at] = o["top_cnt"][at, 0]
        tokens[at] = o["top_tok"][at, :8]
        counts[at] = o["top_cnt"][at, :8]
        filled[at] = True
    cnt_bin = np.searchsorted(COUNT_EDGES, total, side="right")
    pur_bin = np.searchsorted(PURITY_EDGES, top / np.maximum(total, 1), side="right")
    cell = ((1 + level) * (len(COUNT_EDGES) + 1) + cnt_bin) * (len(PURITY_EDGES) + 1) + pur_bin
    cell = np.where(level >= 0, cell, 0).astype(np.int16)
    return cell, tokens, weights(counts)


def pack_rows(cell: np.ndarray, tokens: np.ndarray, w: np.ndarray) -> np.ndarray:
    """gpu_val_stats.cu variant_rows' int32 [N, 9] packing: cell, 4 x (two tokens), 4 x (two weights)."""
    n = len(cell)
    rows = np.zeros((n, 9), np.int32)
    rows[:, 0] = cell.astype(np.int32)
    rows[:, 1:5] = tokens.view(np.int32).reshape(n, 4) if tokens.flags.c_contiguous else \
        np.ascontiguousarray(tokens).view(np.int32).reshape(n, 4)
    rows[:, 5:9] = np.ascontiguousarray(w).view(np.int32).reshape(n, 4)
    return rows


def features(counts: np.ndarray):
    """mix.py features (:22-31): counts int32 [3, L, n] (tot as uint32 bits, dist, cnt) -> tot, dist, cnt (float32
    [n, L]), bin index (int64), sparse index (int64). floor(log2) is of the float32 total, as the reference computes
    it (a correctly rounded float32 log2: the float64 log2 rounded to float32)."""
    tot = (counts[0].T.astype(np.int64) & 0xFFFFFFFF).astype(np.float32)
    dist = counts[1].T.astype(np.float32)
    cnt = np.minimum(counts[2].T.astype(np.float32), tot)
    L = tot.shape[1]
    lg = np.log2(np.maximum(tot, np.float32(1)).astype(np.float64)).astype(np.float32)
    b = np.clip(np.floor(lg), 0, NB - 1).astype(np.int64) + NB * np.arange(L)
    s = (dist == 1).astype(np.int64) + 2 * np.arange(L) + NB * L
    return tot, dist, cnt, b, s


def table_rows(per_level: dict[int, Outputs], row_levels, buckets, entries: int = 8):
    """exact_match/src/count_table.rs query_rows (:338-404): per position the deepest of `row_levels` whose context
    occurred -> (cell int16 [N], next uint16 [N, entries], weights uint16 [N, entries], level int8 [N]); weights are
    round_ties_even(count / sum of the kept counts * 65535) in float64."""
    n = len(next(iter(per_level.values()))["tot"])
    cell = np.zeros(n, np.int16)
    nxt = np.zeros((n, entries), np.uint16)
    w = np.zeros((n, entries), np.uint16)
    level = np.full(n, -1, np.int8)
    filled = np.zeros(n, bool)
    for k in sorted(row_levels, reverse=True):
        o = per_level[k]
        b = list(buckets).index(k)
        at = np.flatnonzero((o["tot"] > 0) & ~filled)
        total = o["tot"][at].astype(np.float64)
        top1 = o["top_cnt"][at, 0].astype(np.float64)
        count_bin = np.searchsorted(COUNT_EDGES, total, side="right")
        purity = np.searchsorted(PURITY_EDGES, top1 / total, side="right")
        cell[at] = ((1 + b) * (len(COUNT_EDGES) + 1) + count_bin) * (len(PURITY_EDGES) + 1) + purity
        kept = o["top_cnt"][at, :entries].astype(np.float64)
        w[at] = np.round(kept / kept.sum(1, keepdims=True) * WEIGHT_ONE).astype(np.uint16)
        nxt[at] = o["top_tok"][at, :entries]
        level[at] = b
        filled[at] = True
    return cell, nxt, w, level


ROW_LEVELS = (6, 10, 20)
ROW_K = 8


def record_rows(tot_rows: np.ndarray, top_tok: np.ndarray, top_cnt: np.ndarray):
    """build.py counts() rows (:341-387). tot_rows uint32 [3, N] (the totals at ROW_LEVELS), top_tok uint16 [3, N, 8],
    top_cnt uint32 [3, N, 8] -> (row_cells int32 [N], row_entries int32 [N, 8])."""
    tc = top_cnt.astype(np.int64)
    tt = top_tok.astype(np.int64)
    top = np.maximum(tc[:, :, :1], 1)
    w = np.where(top > 32767, (tc * 32767 + top - 1) // top, tc)
    entries = np.where(tc > 0, tt | (w << 16), 0).astype(np.int64)
    entries = ((entries + (1 << 31)) % (1 << 32) - (1 << 31)).astype(np.int32)  # int32 wrap, as torch's int32 math
    row_top = np.minimum(tc[:, :, 0], (1 << 31) - 1)
    tot = tot_rows.astype(np.int64)
    n = tot.shape[1]
    depth = ((tot > 0) * np.arange(1, 4)[:, None]).max(0) - 1
    sel = np.maximum(depth, 0)
    pos = np.arange(n)
    total = tot[sel, pos].astype(np.float64)
    share = row_top[sel, pos].astype(np.float64) / np.maximum(total, 1)
    count_bin = sum((total >= e).astype(np.int64) for e in COUNT_EDGES)
    purity = sum((share >= e).astype(np.int64) for e in PURITY_EDGES)
    cell = (((1 + depth) * 7 + count_bin) * 6 + purity) * (depth >= 0)
    ent = np.where((depth >= 0)[:, None], entries[sel, pos], 0)
    return cell.astype(np.int32), ent.astype(np.int32)


def batch_rows(row_cells: np.ndarray, row_entries: np.ndarray, at: int, n: int, capacity: int) -> np.ndarray:
    """build.py batch_rows (:390-403)."""
    cell, e = row_cells[at : at + n], row_entries[at : at + n]
    pos, k = np.nonzero(e != 0)
    m = len(pos)
    if m > capacity:
        raise AssertionError(f"{m} candidates overflow the rows' {capacity} entries")
    rows = np.zeros(n + 2 * capacity, np.int32)
    rows[:n] = cell
    ent = rows[n:].reshape(-1, 2)
    ent[:, 0] = np.arange(capacity, dtype=np.int32) % n
    ent[:m, 0] = pos
    ent[:m, 1] = e[pos, k]
    return rows
