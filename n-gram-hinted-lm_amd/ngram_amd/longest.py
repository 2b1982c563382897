"""Longest exact suffix match of query positions against a training corpus on one MI355X (configuration c5; the
match-length notion of exact_match/src/kgram.rs kgram_stats :38-56, 237-278, taken up to k = 64 by
src/retrieval_blog_post/kgram.py :16, 84-108): per query position i the largest k <= cap whose k-context
x[i-k+1..i] is valid (within its segment) and occurred in the corpus (k tokens within one shard followed by a token
of that shard), that context's most frequent next token (count descending, then token ascending) and its count; 0, 0,
0 if not even the 1-context occurred.

Two phases, both on libngram_amd.so. Existence, k = 1, 2, ...: the query contexts of the positions still matching
(a query index per level over the list of positions still matching), the corpus positions whose (k-1)-context
matched (a hit bitmap while dense, then a position list) probed for their k-context (ng_scan_exist: a bitmap, a
per-context hit bit and each hit position's context id, no counting), until no position matches; once the lists
shrink slowly, the remaining levels run as one stream of launches with device-side counts (no host sync per level).
A match is monotone in k (kgram.rs:12-15), so each position's length is its last matching level. Then counting,
only for each position's final context: a bitmap level's hit positions whose stored context id is final emit their
(context, next) events (ng_scan_ids_emit: no second query index or probe); a list level's final contexts get a query
index and its listed positions are probed, the list levels counted together. The events are partitioned and counted
in LDS (partcount.py: no global atomics, so the hot pairs of short contexts cost no serialized chains), each
context's top entry made from its pairs (ng_ctx_summary) and gathered to its positions (ng_pos_summary).

Surfaces: `longest_match(...)` on GPU tensors, and `LongestMatch.create(files, tokens, threads, cpus)` /
`build() -> dict` in cache_ladder's shape (cache_ladder/src/lib.rs:1-8, cache_ladder.pyi)."""

from __future__ import annotations

import os
import time
from types import SimpleNamespace

import numpy as np
import torch


from .data import BOS, HEADER_BYTES, shard_tokens
from .data import pack_layout as layout
from .lib import Lib, i32, u64
from .partcount import (W_MAX, count32, count_events, emit_region, first_digit, key_mbits, pack_events, pbits32_max,
                        runs_fit, summarize, w_bits)
from .qindex import LOAD as QLOAD, TAIL as QTAIL, QueryIndex


def _popcount(lib: Lib, bm: torch.Tensor) -> int:
    c = torch.zeros(1, dtype=torch.int64, device=bm.device)
    lib("popcount", bm, bm.numel(), c)
    return int(c.item())


_RATIO: dict[int, float] = {}  # distinct pairs per counted event at each level, from the last count (sizes partitions)
_WIDE: set = set()  # levels whose 32-bit count overflowed its escape table: counted by the 64-bit path
# each existence level's query contexts per listed position in the last call: sizes the next call's query index for
# its own number of positions
_CONTEXTS: dict[int, float] = {}


def longest_match(tok: torch.Tensor, x: torch.Tensor, avail: torch.Tensor, cap: int = 64, elib: Lib | None = None,
                  lib: Lib | None = None, timing: dict | None = None, query: torch.Tensor | None = None):
    """Per query position (x int16 [N] inputs, avail int32 [N] tokens since the segment start): (length int32,
    next int16 (uint16 bits), count int32 (uint32 bits)) of its longest match <= cap, and per level
    (k, eligible, matched) over the existence phase. `tok`: the corpus laid out with SENT gaps (layout()).
    `query` (bool [N], optional): only these positions are queried (their contexts still read x before them); the
    others get 0, 0, 0."""
    if not 1 <= cap <= 64:
        raise ValueError("cap must be in [1, 64]")
    EVENTS[0] = 0
    elib = elib or Lib()
    lib = lib or Lib()
    dev = x.device
    N, L = x.numel(), tok.numel()
    nwords = L // 32
    grid = torch.cuda.get_device_properties(dev).multi_processor_count * SCAN_BLOCKS_PER_CU
    t0 = time.perf_counter()
    length = torch.zeros(N, dtype=torch.int32, device=dev)
    # the queried positions, as a list; each level keeps the ones still matching (the lists shrink fast)
    sel = avail >= 1 if query is None else (avail >= 1) & query
    act = torch.nonzero(sel).squeeze(1).to(torch.int32)
    # eligible at level k: queried positions with avail >= k (one histogram for every level)
    elig = torch.bincount(avail[act.long()].clamp_max(cap).long(), minlength=cap + 1).flip(0).cumsum(0).flip(0)
    elig = elig.cpu().tolist()
    # each level's hit set (the corpus positions whose k-context is a query context of the level): a bitmap while
    # dense, then, once sparse, a list of positions, which the next level scans instead of every bitmap word
    levels: list[tuple[str, torch.Tensor, int]] = []
    ladder = []
    flags = torch.zeros(2, dtype=torch.int32, device=dev)
    # the prefix rule for the bitmap scans (a device flag, no host sync): with every position queried, a position
    # still active at level k has its predecessor active at level k - 1 (its shorter context occurs wherever the
    # longer one does), so where avail is segment-shaped a level's context also has its prefix among the level before's
    # and a corpus position is probed only where the level before hit it and the position before it. A query mask can
    # leave a predecessor out, so it turns the rule off.
    pre = None
    if query is None:
        pre = torch.empty(1, dtype=torch.int32, device=dev)
        elib("ng_avail_closed", avail, N, pre)
    for k in range(1, cap + 1):
        act = act[avail[act.long()] >= k]
        if act.numel() == 0:
            break
        if levels and levels[-1][0] == "list" and DEVICE_LEVELS:
            # the sparse levels' lists shrink slowly from here on: the remaining levels run without a host sync
            for k2, hl, nh, matched in _exist_device(elib, tok, L, x, avail, act, k, cap, levels[-1][1], length,
                                                    flags, grid):
                levels.append(("list", hl, nh))
                ladder.append((k2, int(elig[k2]), matched))
            break
        prev = levels[-1] if levels else None
        if prev is None and k == 1:
            # level 1: a 1-context's id is its token, so no query table (ng_scan_tok1 holds the query tokens' set)
            vi = _tok1_index(x, act)
            hit = torch.zeros(2048, dtype=torch.int32, device=dev)
            bm = torch.empty(nwords, dtype=torch.int32, device=dev)
            # no stored ids: a hit's context id is the token before it, which the counting scan reads itself
            elib("ng_scan_tok1", tok, L, vi.member, bm, hit, None, i32(TOK1_GRID))
            levels.append(("bm", bm, _popcount(lib, bm), None, act, vi.ctx_of, vi.ids))
            ctx = vi.ctx_of.long()
            act = act[((hit[ctx >> 5] >> (ctx & 31)) & 1) != 0]
            length[act.long()] = k
            ladder.append((k, int(elig[k]), int(act.numel())))
            del vi, hit, ctx
            continue
        per = _CONTEXTS.get(k)
        vi = QueryIndex(elib, x, avail, k, act, compact=True,
                        expect=None if per is None else int(per * act.numel()) + 1)
        _CONTEXTS[k] = vi.n / max(1, act.numel())
        hit = torch.zeros((vi.ids + 31) // 32, dtype=torch.int32, device=dev)  # a bit per context id
        if prev is not None and (prev[0] == "list" or prev[2] * LIST_DIV < L):
            cand = prev[1] if prev[0] == "list" else _bits_list(elib, prev[1], prev[2])
            hl, nh = _scan_list(elib, tok, L, k, vi, x, cand, hit, 1, flags, grid)
            levels.append(("list", hl, nh))
        else:
            bm = torch.empty(nwords, dtype=torch.int32, device=dev)
            ids = torch.empty(L, dtype=torch.int32, device=dev)  # each hit position's context id, for the counting
            mode = 0 if prev is None or prev[2] * 2 > L else 2  # a lane per position while the gate is dense
            elib("ng_scan_exist", tok, L, i32(k), None if prev is None else prev[1], bm, vi.table, u64(vi.cap),
                 vi.rep, x, hit, ids, flags, i32(grid), i32(mode), pre)
            levels.append(("bm", bm, _popcount(lib, bm), ids, act, vi.ctx_of, vi.ids))
        ctx = vi.ctx_of.long()
        c = ctx.clamp_min(0)
        act = act[(ctx >= 0) & (((hit[c >> 5] >> (c & 31)) & 1) != 0)]
        length[act.long()] = k
        ladder.append((k, int(elig[k]), int(act.numel())))
        del vi, hit, ctx
    if timing is not None:
        torch.cuda.synchronize()
        timing["exist"] = timing.get("exist", 0.0) + time.perf_counter() - t0
        t0 = time.perf_counter()
    nxt = torch.zeros(N, dtype=torch.int16, device=dev)
    cnt = torch.zeros(N, dtype=torch.int32, device=dev)
    # each level's final positions (those whose longest match has that length), grouped by one sort
    qpos = torch.nonzero(sel).squeeze(1)
    qlen = length[qpos]
    order = torch.argsort(qlen, stable=True)
    qpos, qlen = qpos[order].to(torch.int32), qlen[order]
    bounds = torch.searchsorted(qlen, torch.arange(len(levels) + 2, device=dev, dtype=torch.int32)).cpu().tolist()
    batch: list = []  # list levels waiting to be counted together: (k, final positions, index)
    batch_ev = 0
    for k in range(1, len(levels) + 1):
        kind, hs, nh = levels[k - 1][:3]
        if kind == "bm":  # counted from the context ids the existence scan stored: no second query index or probe
            _count_ids(elib, lib, tok, L, levels[k - 1], k, length, flags, grid, nxt, cnt)
            levels[k - 1] = levels[k - 1][:3]
            continue
        fpos = qpos[bounds[k] : bounds[k + 1]]
        m = fpos.numel()
        if m == 0:
            continue
        if kind == "list":  # a sparse level: counted with the other list levels, one count for all
            # its index is not checked here (no host wait per level): the batch reads every level's counters with its
            # event total, and is counted again on indexes checked as they are built if an insert found no slot
            vi = QueryIndex(elib, x, avail, k, fpos, compact=True, expect=m, defer=True)
            batch.append((k, fpos, vi))
            batch_ev += nh
            if batch_ev >= BATCH_EVENTS:
                _count_batch(elib, lib, tok, L, x, avail, batch, levels, flags, grid, nxt, cnt)
                batch, batch_ev = [], 0
            continue
        vi = QueryIndex(elib, x, avail, k, fpos, compact=True)
        # the level's hit positions probed against the final contexts; their hits emitted, partitioned and counted in
        # LDS, then each final context's top entry
        flags.zero_()
        ev, n_ev = _scan_list(elib, tok, L, k, vi, x, hs, None, 0, flags, grid)
        if int(flags[0].item()) & 4:
            raise RuntimeError(f"k={k}: an emit region overflowed")
        c = count_events(elib, lib, ev, n_ev, vi.ids, _RATIO.get(k, 1.0), presort="ctx")
        n_ev = c.n_ev
        EVENTS[0] += n_ev
        del ev
        _RATIO[k] = c.U / max(1, n_ev)
        o_tok = torch.zeros(m, dtype=torch.int16, device=dev)
        o_cnt = torch.zeros(m, dtype=torch.int32, device=dev)
        if c.cb:
            sm = summarize(elib, lib, c, vi.ids, 1)
            rec, dist = sm.rec, sm.dist
            o_tot = torch.empty(m, dtype=torch.int32, device=dev)
            o_dist = torch.empty(m, dtype=torch.int32, device=dev)
            o_tc = torch.empty(m, dtype=torch.int32, device=dev)
            elib("ng_pos_summary", vi.ctx_of, m, 0, vi.ids, None, rec, dist, None, None, i32(1), i32(1), i32(0),
                 o_tot, o_dist, o_tc, o_tok, o_cnt, None, None)
            del rec, dist, o_tot, o_dist, o_tc
        else:  # unpacked pairs: sorted by key, per-context top entry by selection
            _top1_unpacked(elib, lib, vi, c, x, o_tok, o_cnt)
        nxt[fpos.long()] = o_tok
        cnt[fpos.long()] = o_cnt
        del vi, c, o_tok, o_cnt
    if batch:
        _count_batch(elib, lib, tok, L, x, avail, batch, levels, flags, grid, nxt, cnt)
    if timing is not None:
        torch.cuda.synchronize()
        timing["count"] = timing.get("count", 0.0) + time.perf_counter() - t0
        timing["events"] = float(EVENTS[0])
    return length, nxt, cnt, ladder


SCAN_BLOCKS_PER_CU = 32  # scan blocks per compute unit
TOK1_GRID = 2048  # level 1's scan blocks (each ORs its hit words into the level's once)
EVENTS = [0]  # (context, next) events the last longest_match counted (its counting phase), for its timing dict
DEVICE_LEVELS = True  # the existence phase's levels after the second list level run without host syncs
LONG_FIRST = 8  # the device levels try level cap first when at least this many levels lie between
BATCH_EVENTS = 1 << 28  # list levels counted together until their listed positions reach this
LIST_DIV = 64  # a level's hits go to a position list once fewer than L / LIST_DIV (8 B each against L / 8 bitmap bytes)


def _exist_device(elib: Lib, tok, L: int, x, avail, act, k0: int, cap: int, cand, length, flags, grid: int):
    """Levels k0..cap of the existence phase as one stream of launches with no host sync (ng_query_index_dev,
    ng_scan_list_dev, ng_seg_offsets / ng_seg_gather, ng_act_next), every buffer sized by level k0's active
    positions (act, already those with avail >= k0) and candidates (cand: the corpus positions that matched k0 - 1),
    which bound every later level's. One sync at the end reads each level's sizes; the levels are those whose active
    list was not empty, as the host loop's. Returns [(k, hit list, its length, matched positions)].

    With LONG_FIRST or more levels to go, level `cap` is tried first (the cap round): a position whose cap-token
    context occurs matches every level below it too (a context's suffixes occur wherever it does), so it is done at
    length cap, and the levels in between are walked by the others only. Their hit lists then hold only those
    positions' contexts' occurrences, and level cap's is the round's. The long copies of a corpus make most of the
    deep levels' positions such ones: they would otherwise be probed, and their occurrences listed, at every level."""
    dev = x.device
    n0, nc0 = int(act.numel()), int(cand.numel())
    qcap = int(n0 / QLOAD) + 1024
    slots = qcap + QTAIL
    table = torch.empty(slots, dtype=torch.int64, device=dev)
    rep = torch.empty(slots, dtype=torch.int32, device=dev)
    ctx_of = torch.empty(max(n0, 1), dtype=torch.int32, device=dev)
    hit = torch.empty((slots + 31) // 32, dtype=torch.int32, device=dev)
    acts = [act.contiguous(), torch.empty(max(n0, 1), dtype=torch.int32, device=dev)]
    nlev = cap - k0 + 1
    counters = torch.zeros((nlev, 3), dtype=torch.int64, device=dev)
    sizes = torch.zeros((nlev, 3), dtype=torch.int64, device=dev)  # per level: active, matched, kept for the next
    g = max(1, min(grid, -(-max(nc0, 1) // 256)))
    R = -(-max(nc0, 1) // (g * 256)) * 256
    regions = torch.empty(g * R, dtype=torch.int64, device=dev)
    ev_count = torch.empty(g, dtype=torch.int32, device=dev)
    n_act = torch.tensor([n0], dtype=torch.int64, device=dev)
    n_cand = torch.tensor([nc0], dtype=torch.int64, device=dev)
    flags.zero_()
    first = cap - k0 >= LONG_FIRST
    if first:  # the cap round: the positions matching level cap are done; the others go on from level k0
        counters_cap = torch.zeros(3, dtype=torch.int64, device=dev)
        split = torch.zeros(2, dtype=torch.int64, device=dev)  # positions going on, positions done at length cap
        elib("ng_query_index_dev", x, avail, acts[0], n_act, n0, i32(cap), table, u64(qcap), u64(slots), rep, ctx_of,
             counters_cap)
        hit.zero_()
        elib("ng_scan_list_dev", tok, i32(cap), cand, n_cand, nc0, table, u64(qcap), rep, x, hit, i32(1), regions,
             u64(R), ev_count, flags, i32(g), u64(0))
        offs = torch.empty(g + 1, dtype=torch.int64, device=dev)
        elib("ng_seg_offsets", ev_count, g, offs)
        hl_cap = torch.empty(max(nc0, 1), dtype=torch.int64, device=dev)
        elib("ng_seg_gather", regions, None, u64(R), None, ev_count, g, offs, hl_cap, None)
        elib("ng_act_split", acts[0], n_act, n0, ctx_of, hit, i32(cap), length, acts[1], split[0:1], split[1:2])
        nh_cap, n_act = offs[g:], split[0:1]
        acts.reverse()
    out = []
    for j, k in enumerate(range(k0, cap if first else cap + 1)):
        cur, nxt = acts[j % 2], acts[(j + 1) % 2]
        sizes[j, 0:1].copy_(n_act)
        elib("ng_query_index_dev", x, avail, cur, n_act, n0, i32(k), table, u64(qcap), u64(slots), rep, ctx_of,
             counters[j])
        hit.zero_()
        elib("ng_scan_list_dev", tok, i32(k), cand, n_cand, nc0, table, u64(qcap), rep, x, hit, i32(1), regions,
             u64(R), ev_count, flags, i32(g), u64(0))
        offs = torch.empty(g + 1, dtype=torch.int64, device=dev)
        elib("ng_seg_offsets", ev_count, g, offs)
        hl = torch.empty(max(nc0, 1), dtype=torch.int64, device=dev)
        elib("ng_seg_gather", regions, None, u64(R), None, ev_count, g, offs, hl, None)
        elib("ng_act_next", cur, n_act, n0, ctx_of, hit, avail, i32(k), length, nxt, sizes[j, 2:3], sizes[j, 1:2])
        out.append((k, hl, offs[g:]))
        cand, n_cand, n_act = hl, offs[g:], sizes[j, 2:3]
    if first:
        out.append((cap, hl_cap, nh_cap))
        counters = torch.cat([counters, counters_cap[None]])
        sizes[-1, 1:2].copy_(split[1:2])
    host = sizes.cpu().tolist()
    nhs = torch.cat([o for _, _, o in out]).cpu().tolist()
    c = counters.cpu()
    if int(flags[0].item()) & 4:
        raise RuntimeError(f"levels {k0}..{cap}: an emit region overflowed")
    if int(c[:, 1].max()):
        raise RuntimeError(f"levels {k0}..{cap}: a query index was too small for its contexts")
    if int(c[:, 2].max()):
        raise RuntimeError(f"levels {k0}..{cap}: query positions collide with another context's key")
    done = host[-1][1] if first else 0  # the positions done at length cap: active and matched at every level
    if first:  # level cap's active positions: the others' that reached it, and the cap round's
        host[-1][0] = host[-2][2] if len(host) > 1 else 0
    res = []
    for (k, hl, _), nh, (n_k, matched, _) in zip(out, nhs, host):
        if k < cap:
            n_k, matched = n_k + done, matched + done
        else:
            n_k += done if first else 0
        if n_k == 0:
            break
        res.append((k, hl[:nh], nh, matched))
    return res


def _tok1_index(x: torch.Tensor, act: torch.Tensor) -> SimpleNamespace:
    """Level 1's index without a table: each listed position's context id is its token (x[act], ids 0..65535), and
    `member` (int32 [2048]) holds bit t for each token t among them."""
    dev = x.device
    ctx_of = x[act.long()].to(torch.int32) & 0xFFFF
    seen = torch.zeros(65536, dtype=torch.bool, device=dev)
    seen[ctx_of.long()] = True
    w = (seen.view(2048, 32).to(torch.int64) << torch.arange(32, device=dev)).sum(1)
    member = torch.where(w >= 1 << 31, w - (1 << 32), w).to(torch.int32)  # the words' bits, as int32
    return SimpleNamespace(ctx_of=ctx_of, ids=65536, member=member)


def _count_ids(elib: Lib, lib: Lib, tok, L: int, level: tuple, k: int, length, flags, grid: int, nxt, cnt) -> None:
    """The counting phase of a bitmap level from what its existence scan kept: the hit bitmap, each hit position's
    context id (None at level 1 by token: the token before the position), and the level's active positions with their
    context ids. The final contexts (those of the positions
    whose match ends at k) are marked in a bit set; the hit positions of final contexts emit their (context, next)
    events (ng_scan_ids_emit), which are partitioned, counted and summarized per context (top entry), then gathered
    to the final positions."""
    _, bm, nh, ids, act, ctx_of, n_ids = level
    dev = bm.device
    fin = length[act.long()] == k
    fids = ctx_of[fin]
    fpos = act[fin].long()
    m = fids.numel()
    if m == 0:
        return
    final = torch.zeros((n_ids + 31) // 32, dtype=torch.int32, device=dev)
    elib("ng_mark_bits", fids, m, final)
    R = emit_region(L, grid)
    regions = torch.empty(grid * R, dtype=torch.int64, device=dev)
    ev_count = torch.empty(grid, dtype=torch.int32, device=dev)
    _, W = w_bits(n_ids)
    if W <= W_MAX and k not in _WIDE:  # the 32-bit count (pairs32.hip), as the level pipeline's
        d1 = first_digit(W)
        dhist = torch.empty((1 << d1) * grid, dtype=torch.int32, device=dev)
        flags.zero_()
        elib("ng_scan_ids_emit", tok, L, bm, ids, final, regions, u64(R), ev_count, flags, i32(grid), dhist, grid,
             i32(W), i32(d1), i32(key_mbits(W) if runs_fit(n_ids, 1) else W))
        if _count32_final(elib, (regions, R, ev_count, dhist, grid, flags), n_ids, k, fids, fpos, m, nxt, cnt):
            return
        _WIDE.add(k)  # its escape table overflowed: this level takes the 64-bit count from now on
    dhist = torch.empty(256 * grid, dtype=torch.int32, device=dev)
    flags.zero_()
    elib("ng_scan_ids_emit", tok, L, bm, ids, final, regions, u64(R), ev_count, flags, i32(grid), dhist, grid, i32(0),
         i32(0), i32(0))
    try:  # the scan's flags read with the event total
        c = count_events(elib, lib, None, 0, n_ids, _RATIO.get(k, 1.0),
                         seg=(regions, R, ev_count, dhist, grid, flags), presort="ctx")
    except RuntimeError as e:
        raise RuntimeError(f"k={k}: {e}") from None
    del regions
    _RATIO[k] = c.U / max(1, c.n_ev)
    EVENTS[0] += c.n_ev
    o_tok = torch.zeros(m, dtype=torch.int16, device=dev)
    o_cnt = torch.zeros(m, dtype=torch.int32, device=dev)
    if c.cb:
        sm = summarize(elib, lib, c, n_ids, 1)
        o = [torch.empty(m, dtype=torch.int32, device=dev) for _ in range(3)]
        elib("ng_pos_summary", fids, m, 0, n_ids, None, sm.rec, sm.dist, None, None, i32(1), i32(1), i32(0), o[0], o[1],
             o[2], o_tok, o_cnt, None, None)
    else:  # unpacked pairs: sorted by key, per-context top entry by selection
        _top1_unpacked(elib, lib, SimpleNamespace(ctx_of=fids, ids=n_ids), c, None, o_tok, o_cnt)
    nxt[fpos] = o_tok
    cnt[fpos] = o_cnt


def _count32_final(elib: Lib, seg: tuple, n_ids: int, k: int, fids, fpos, m: int, nxt, cnt) -> bool:
    """The 32-bit count of a level's final contexts' events (seg: ng_scan_ids_emit's W-bit regions), their top entry
    gathered to the final positions; an overfull partition is counted again with one more partition bit. False (the
    caller takes the 64-bit count) when the escape table overflowed."""
    dev = fids.device
    min_pbits = 0
    while True:
        c = count32(elib, seg, n_ids, 1, None, None, _RATIO.get(k, 1.0), min_pbits=min_pbits,
                    mbits=key_mbits(w_bits(n_ids)[1]) if runs_fit(n_ids, 1) else None)
        n_ev, n_u, fl, scan = c.stat[:4].cpu().tolist()
        if int(seg[5][0].item()) & 4:
            raise RuntimeError(f"k={k}: an emit region overflowed")
        if fl & 4:
            raise RuntimeError(f"k={k}: a total does not fit uint32")
        if fl & 2:
            return False
        if fl & 1 and c.pbits < pbits32_max(n_ids):
            min_pbits = c.pbits + 1
            continue
        if fl & 1:
            return False
        break
    _RATIO[k] = n_u / max(1, n_ev)
    EVENTS[0] += n_ev
    o = [torch.empty(m, dtype=torch.int32, device=dev) for _ in range(3)]
    o_tok = torch.zeros(m, dtype=torch.int16, device=dev)
    o_cnt = torch.zeros(m, dtype=torch.int32, device=dev)
    elib("ng_pos_summary", fids, m, 0, n_ids, None, c.rec, c.dist, None, None, i32(1), i32(1), i32(0), o[0], o[1],
         o[2], o_tok, o_cnt, None, None)
    nxt[fpos] = o_tok
    cnt[fpos] = o_cnt
    return True


def _bits_list(elib: Lib, bm: torch.Tensor, n: int) -> torch.Tensor:
    """The set positions of a bitmap (n of them) as a u64 list."""
    out = torch.empty(max(n, 1), dtype=torch.int64, device=bm.device)
    total = torch.zeros(1, dtype=torch.int64, device=bm.device)
    elib.cub("ng_bits_list", bm, bm.numel(), out, total, None)
    return out[:n]


def _scan_list(elib: Lib, tok, L: int, k: int, vi, x, cand: torch.Tensor, hit, what: int, flags, grid: int):
    """A level scan of listed corpus positions: hits flagged per context (hit may be None) and emitted as positions
    (what 1) or mixed pair keys (what 0), packed: (list, n)."""
    n = cand.numel()
    g = max(1, min(grid, -(-n // 256)))  # a round of 256 entries per block: as many blocks as fill the GPU
    R = -(-max(n, 1) // (g * 256)) * 256  # a list scan's block emits at most 256 per round
    regions = torch.empty(g * R, dtype=torch.int64, device=cand.device)
    ev_count = torch.empty(g, dtype=torch.int32, device=cand.device)
    elib("ng_scan_sink", tok, L, i32(k), None, None, cand, n, vi.table, u64(vi.cap), vi.rep, x, hit, i32(what),
         regions, u64(R), ev_count, flags, i32(g), i32(0), u64(0))
    out, m = pack_events(elib, regions, R, ev_count, g)
    return out[:m] if what else out, m


def _count_batch(elib: Lib, lib: Lib, tok, L: int, x, avail, batch: list, levels: list, flags, grid: int, nxt,
                 cnt) -> None:
    """The counting phase of several list levels at once: level k's context ids offset by the ids before it in the
    batch, so one partitioned count, one summary and one gather serve them all (per level only its query index and
    its scan: few launches and no host sync per level)."""
    dev = x.device
    bases, n_ids = [], 0
    for _, _, vi in batch:
        bases.append(n_ids)
        n_ids += vi.ids
    cap_ev = sum(levels[k - 1][2] for k, _, _ in batch)  # each listed position emits at most one event
    ev = torch.empty(max(cap_ev, 1), dtype=torch.int64, device=dev)
    at = torch.zeros(1, dtype=torch.int64, device=dev)  # the events packed so far (device side)
    flags.zero_()
    for (k, _, vi), b in zip(batch, bases):
        _, hs, nh = levels[k - 1]
        g = max(1, min(grid, -(-nh // 256)))
        R = -(-max(nh, 1) // (g * 256)) * 256
        regions = torch.empty(g * R, dtype=torch.int64, device=dev)
        ev_count = torch.empty(g, dtype=torch.int32, device=dev)
        elib("ng_scan_sink", tok, L, i32(k), None, None, hs, nh, vi.table, u64(vi.cap), vi.rep, x, None, i32(0),
             regions, u64(R), ev_count, flags, i32(g), i32(0), u64(b << 16))
        offs = torch.empty(g + 1, dtype=torch.int64, device=dev)
        elib("ng_seg_offsets", ev_count, g, offs)
        offs += at
        elib("ng_seg_gather", regions, None, u64(R), None, ev_count, g, offs, ev, None)
        at = offs[g : g + 1].clone()
        del regions, ev_count
    pending = [(k, vi.pending) for k, _, vi in batch if vi.n is None]  # deferred indexes' counters
    got = torch.cat([at, flags[:1].to(torch.int64)] + [c for _, c in pending]).tolist()  # one copy
    n_ev, fl = got[:2]
    if fl & 4:
        raise RuntimeError(f"levels {batch[0][0]}..{batch[-1][0]}: an emit region overflowed")
    for j, (k, _) in enumerate(pending):
        _, over, coll = got[2 + 3 * j : 5 + 3 * j]
        if coll:
            raise RuntimeError(f"k={k}: {coll} query positions collide with another context's key")
        if over:  # an insert found no slot (a walk past its bound): the batch again, its indexes checked
            del ev
            redo = [(k2, f, QueryIndex(elib, x, avail, k2, f, compact=True)) for k2, f, _ in batch]
            return _count_batch(elib, lib, tok, L, x, avail, redo, levels, flags, grid, nxt, cnt)
    key = ("batch", batch[0][0])
    c = count_events(elib, lib, ev, n_ev, n_ids, _RATIO.get(key, 1.0), presort="ctx")
    del ev
    _RATIO[key] = c.U / max(1, n_ev)
    EVENTS[0] += n_ev
    if not c.cb:
        raise RuntimeError(f"levels {batch[0][0]}..{batch[-1][0]}: more large counts than the escape table holds")
    sm = summarize(elib, lib, c, n_ids, 1)
    fpos = torch.cat([f for _, f, _ in batch]).long()
    ctx_of = torch.cat([torch.where(vi.ctx_of >= 0, vi.ctx_of + b, -1) for (_, _, vi), b in zip(batch, bases)])
    m = fpos.numel()
    o_tok = torch.zeros(m, dtype=torch.int16, device=dev)
    o_cnt = torch.zeros(m, dtype=torch.int32, device=dev)
    o_tot = torch.empty(m, dtype=torch.int32, device=dev)
    o_dist = torch.empty(m, dtype=torch.int32, device=dev)
    o_tc = torch.empty(m, dtype=torch.int32, device=dev)
    elib("ng_pos_summary", ctx_of, m, 0, n_ids, None, sm.rec, sm.dist, None, None, i32(1), i32(1), i32(0), o_tot, o_dist,
         o_tc, o_tok, o_cnt, None, None)
    nxt[fpos] = o_tok
    cnt[fpos] = o_cnt


def _top1_unpacked(elib: Lib, lib: Lib, vi, c, x, o_tok, o_cnt) -> None:
    """The final contexts' top entries from unpacked (pair key, count) pairs (compact ctx_of, m entries)."""
    dev = o_tok.device
    m = vi.ctx_of.numel()
    ctx_bits = max(1, (max(vi.ids, 2) - 1).bit_length())
    uk = torch.empty(c.U, dtype=torch.int64, device=dev)
    agg = torch.empty(c.U, dtype=torch.int32, device=dev)
    if c.U:
        lib.cub("sort_pairs", c.pairs, uk, c.counts, agg, c.U, i32(0), i32(16 + ctx_bits))
    start = torch.zeros(vi.ids, dtype=torch.int64, device=dev)
    end = torch.zeros(vi.ids, dtype=torch.int64, device=dev)
    tot = torch.zeros(vi.ids, dtype=torch.int64, device=dev)
    top_tok = torch.zeros(vi.ids, dtype=torch.int16, device=dev)
    top_cnt = torch.zeros(vi.ids, dtype=torch.int32, device=dev)
    lib("seg_bounds", uk, c.U, start, end)
    elib("ng_ctx_topk", uk, agg, start, end, vi.ids, i32(1), tot, top_tok, top_cnt)
    o = [torch.zeros(m, dtype=torch.int32, device=dev) for _ in range(3)]
    tgt = torch.zeros(m, dtype=torch.int16, device=dev)
    elib("ng_pos_gather", vi.ctx_of, m, 0, vi.ids, tgt, uk, agg, start, end, tot, top_tok, top_cnt, None, None, None,
         u64(0), None, i32(1), i32(1), i32(0), o[0], o[1], o[2], o_tok, o_cnt, None)


def _segments(x: torch.Tensor, lib: Lib) -> torch.Tensor:
    n = x.numel()
    idx = torch.arange(n, device=x.device)
    start = (x.to(torch.int32) & 0xFFFF) == BOS
    start[:1] = True
    seg = torch.empty_like(idx)
    if n:
        lib.cub("inclusive_max", torch.where(start, idx, torch.zeros_like(idx)), seg, n)
    return (idx - seg + 1).to(torch.int32)


class LongestMatch:
    """The longest match as a ladder rung (cache_ladder's interface, cache_ladder/src/lib.rs:1-8): create(files,
    tokens, threads, cpus) reads the training shards and the query stream (`tokens`: the inputs, then the last one's
    next token) before the clock; build() runs the match on the clock and returns its timings (seconds) and sizes;
    afterwards `length`, `next` (uint16) and `count` (uint32) hold the per-position results (numpy)."""

    def __init__(self):
        raise TypeError("use LongestMatch.create(files, tokens, threads, cpus)")

    @staticmethod
    def create(files: list, tokens, threads: int = 1, cpus: list[int] = (), cap: int = 64) -> "LongestMatch":
        self = object.__new__(LongestMatch)
        arrays = []
        for f in files:
            if isinstance(f, (str, bytes, os.PathLike)):
                n = shard_tokens(f)
                arrays.append(np.fromfile(f, dtype="<u2", count=n, offset=HEADER_BYTES))
            else:
                arrays.append(np.ascontiguousarray(f, dtype=np.uint16))
        q = np.ascontiguousarray(tokens, dtype=np.uint16)
        if not arrays or len(q) < 2 or int(q.max()) > BOS or any(len(a) and int(a.max()) > BOS for a in arrays):
            raise ValueError("need training shards and 2+ valid query tokens")
        sizes = [len(a) for a in arrays]
        starts, L = layout(sizes)
        dev = torch.device("cuda", torch.cuda.current_device())
        self.tok = torch.full((L,), -1, dtype=torch.int16, device=dev)
        for a, st in zip(arrays, starts):
            if len(a):
                self.tok[st : st + len(a)].copy_(torch.from_numpy(a.view(np.int16)))
        self.x = torch.from_numpy(q[:-1].view(np.int16).copy()).to(dev)
        self.cap = cap
        self.elib = self.lib = Lib()
        self.avail = _segments(self.x, self.lib)
        self.tokens = int(sum(sizes))
        torch.cuda.synchronize()
        return self

    def build(self) -> dict:
        timing: dict = {}
        t0 = time.perf_counter()
        length, nxt, cnt, ladder = longest_match(self.tok, self.x, self.avail, self.cap, self.elib, self.lib, timing)
        torch.cuda.synchronize()
        timing["total"] = time.perf_counter() - t0
        self.length = length.cpu().numpy().view(np.uint32)
        self.next = nxt.cpu().numpy().view(np.uint16)
        self.count = cnt.cpu().numpy().view(np.uint32)
        self.ladder = ladder
        timing["levels"] = float(len(ladder))
        return timing
