"""The engine's level pipeline: query-filtered exact counts of every (context, next token) pair of a device-resident
token buffer, level after level, and the per-position outputs. Both host surfaces run on it: the record's CountBuild
(record_367_gpu_counts/track_1_short/counts/build.py:261-388) and the validation statistics' build
(old_records/gpu_val_stats.py _run :701-1232). No counterpart in the reference's libraries: there a level's hits are
counted with global atomics in one hash table and ranked by a second sort; here

  1. the level's query index (ng_query_index, qindex.py) holds only the query positions whose previous level's context
     occurred (a k-context occurs only where its (k-1)-suffix does);
  2. the level's scan (ng_scan_emit: every position, or only those its shard's previous level hit) appends each hit's
     mix64(context id << 16 | next) to its block's own region, no global atomic, and makes the hit bitmap that gates
     the next level; a level behind a sparse one lists the previous hits first (ng_bits_list) and probes the list.
     When the query contexts are closed under prefixes (ng_avail_closed: segment-shaped avail, checked on the device)
     a position is probed only if the previous level hit both there and one position earlier: a k-context occurs
     only where its (k-1)-suffix and its (k-1)-prefix both do. The scans are bound by random-line requests, so every
     position the rule drops is a request saved;
  3. the events are hash-partitioned by a radix pass straight from the regions and counted partition by partition in
     LDS (partcount.count_events), which also answers each query position's (context, target) count;
  4. the distinct pairs, packed one word each, are sorted by context and summarized per present context
     (ng_ctx_summary: total, pairs, top entries); with a TOP rule the contexts with more than `cnt_top` pairs get the
     cnt_top-th largest score (ng_ctx_kth);
  5. per query position its context's record gives tot, dist, the target's count (if ranked within cnt_top) and the
     top entries (ng_pos_summary), and the level's mask bit.

Per-level sizes from one build are kept (context counts, events, distinct pairs per event, hit densities) and size the
next build of the same inputs."""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch

from . import partcount
from .lib import Lib, i32, u64
from .partcount import (W_MAX, check_summary, count32, count_events, emit_region, first_digit, key_mbits, summarize,
                        w_bits)
from .qindex import EXPECT_MARGIN, LOAD as QLOAD, TAIL as QTAIL, QueryIndex

SCAN_BLOCKS_PER_CU = 8  # level-scan blocks (grid-stride) per compute unit (c3 sweep: 8 fastest of 4-32)
LIST_DENSITY = 0.05  # a level behind a sparser one probes the previous hits as a position list (c3 sweep)
DENSE_LOAD = 0.22  # query-table load of a level probed at every position, where it keeps the count's layout (c3,
# levels 2 and 3: 65.3-65.5 against 66.0-66.2 ms a step; 0.4-0.6 at level 3 made its scan slower, not faster, although
# its table then fitted the 256 MB cache)
SEEN_MARGIN = 1.05  # room for a level's query positions listed on the device: this times the last build's count
# (at least 1: a list that overflowed is listed again in room for the count it found)
TOPS = (1, 2, 4, 8)  # the record widths ng_ctx_summary writes


def _record_width(want: int) -> int:
    return next(t for t in TOPS if t >= max(want, 1))


@dataclass
class LevelOutputs:
    """One build's outputs: counts int32 [3, len(levels), N] (tot and cnt as uint32 bits, dist <= 65535), with topk
    the top entries per level and position (int16 [L, N, topk], int32 [L, N, topk]), with mask the levels whose context
    occurred (bit li of int32 [N]), and for each kept level (ctx_of int32 [N], records CtxRecord<8> int32 [ids, 16])."""

    counts: torch.Tensor
    top_tok: torch.Tensor | None = None
    top_cnt: torch.Tensor | None = None
    mask: torch.Tensor | None = None
    kept: dict = field(default_factory=dict)
    info: dict = field(default_factory=dict)


class LevelBuild:
    """Exact counts of `levels` (ascending k) over the shards laid out in `tok` (int16 [L], data.pack_layout's
    starts/sizes). `level_shards`: per level, how many leading shards it counts (default: all). `ready`: per shard an
    event its first scan waits for (its copy from the host), or None for resident tokens."""

    def __init__(self, tok: torch.Tensor, sizes: list[int], starts: list[int], levels, level_shards: dict | None = None,
                 ready: list | None = None, elib: Lib | None = None):
        self.levels = tuple(levels)
        if not self.levels or list(self.levels) != sorted(set(self.levels)) or self.levels[0] < 1:
            raise ValueError(f"levels must ascend from >= 1: {self.levels}")
        self.tok, self.sizes, self.starts = tok, list(sizes), list(starts)
        self.L = int(tok.numel())
        ls = level_shards or {}
        self.level_shards = {k: min(len(sizes), ls.get(k, len(sizes))) for k in self.levels}
        self.ready = ready
        self.elib = elib or Lib()
        # sizes learnt from the last build: hit density, events, query contexts, distinct pairs per event
        self.density: dict[int, float] = {}
        self.events_of: dict[int, int] = {}
        self.contexts_of: dict[int, int] = {}
        self.dratio: dict[int, float] = {}
        self.kernel_events: list = []
        self.host_s = {"index": 0.0, "scan": 0.0, "count": 0.0}
        self._plist = None
        self._no_bm = None  # the level whose list scan sets no hit bits (the last one, without hit statistics)
        self.wide: set = set()  # levels counted by the 64-bit path (count_events): their 32-bit count overflowed
        self.min_pbits: dict[int, int] = {}  # per level, partition bits the 32-bit count found too few, plus one
        self.seen_of: dict[int, int] = {}  # per level, the query positions whose previous level's context occurred
        self.reruns = 0  # builds run again (a size learnt from an earlier build fell short), over this engine's life

    def _event(self, name: str, k: int, n: int, mode: int = -1):
        """A pair of timing events around a launch on the current stream, kept in kernel_events as (name, k, n, e0,
        e1, mode): n the items the launch covers (a scan: the positions of its range), mode a scan's (see _mode)."""
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        self.kernel_events.append((name, k, n, e0, e1, mode))
        return e0, e1

    def _wait(self, i: int) -> None:
        if self.ready is not None and self.ready[i] is not None:
            torch.cuda.current_stream().wait_event(self.ready[i])

    def build(self, x: torch.Tensor, tgt: torch.Tensor, avail: torch.Tensor, *, topk: int = 0,
              cnt_top: int | None = None, keep=(), with_mask: bool = False, stats: bool = False,
              _defer: bool = True) -> LevelOutputs:
        """Counts of every level for the N query positions (x int16 [N], tgt int16 [N], avail int32 [N]). `topk`: also
        each position's context's first topk entries; `cnt_top`: the TOP rule (cnt only if the target ranks below it);
        `keep`: levels whose records are returned (top-8); `stats`: each level's corpus hits in info."""
        dev, N, elib = self.tok.device, x.numel(), self.elib
        want_stats = stats
        self.kernel_events = []
        self.grid = torch.cuda.get_device_properties(dev).multi_processor_count * SCAN_BLOCKS_PER_CU
        nwords = self.L // 32
        # the levels' hit bitmaps: a dense, sparse or compact scan writes every word of its range, so only a list
        # scan's range is zeroed (before it sets its bits); hit statistics count whole bitmaps, so they zero them all
        bms = {k: torch.empty(nwords, dtype=torch.int32, device=dev) for k in self.levels}
        if want_stats:
            for bm in bms.values():
                elib.fill(bm, 0)
        # no level reads the last one's bitmap (only hit statistics do): its list scan sets no bits
        self._no_bm = None if want_stats else self.levels[-1]
        # every level's ng_pos_summary writes all N positions of its rows (zeros where the context is absent): no fill
        res = LevelOutputs(torch.empty((3, len(self.levels), N), dtype=torch.int32, device=dev))
        self._pre = torch.empty(1, dtype=torch.int32, device=dev)  # the prefix rule's device flag
        elib("ng_avail_closed", avail, N, self._pre)
        if topk:
            res.top_tok = torch.empty((len(self.levels), N, topk), dtype=torch.int16, device=dev)
            res.top_cnt = torch.empty((len(self.levels), N, topk), dtype=torch.int32, device=dev)
        if with_mask:
            res.mask = elib.zeros(N, torch.int32, dev)
        G = self.grid
        R = max([emit_region((n + 31) // 32 * 32, G) for n in self.sizes] or [8192])
        span = self.starts[-1] + (self.sizes[-1] + 31) // 32 * 32 - self.starts[0] if self.sizes else 0
        # room for one region per shard and block, or for one scan over every shard (a list scan's regions included)
        n_reg = max(len(self.sizes) * G * R, G * emit_region(span, G), G * (-(-max(span, 1) // (G * 256)) * 256))
        regions = torch.empty(n_reg, dtype=torch.int64, device=dev)
        out = res.counts
        deferred = []  # summarize's checks, read once after every level
        checks32 = []  # the 32-bit counts' sizes and flags, likewise
        pending = []  # query indexes sized from the last build's context counts, checked once after every level
        # every level's device-side results in one tensor, read with one copy after the last level: per level the
        # 32-bit count's events, pairs and flags, the scan's flags, the listed query positions, the index's counters
        stats = elib.zeros((len(self.levels), 8), torch.int64, dev)
        hit_bits = torch.empty((N + 63) // 64 * 2, dtype=torch.int32, device=dev)  # a level's occurred contexts' positions
        for li, k in enumerate(self.levels):
            t0 = time.perf_counter()
            prev = self.levels[li - 1] if li else None
            seen = seen_n = None
            seen_cap = 0
            if prev is not None and self.level_shards[k] <= self.level_shards[prev]:
                if cnt_top is None and k not in self.wide and k in self.seen_of and _defer:
                    # listed on the device, sized from the last build's count: no host wait (checked after the last
                    # level; a list that came out longer than its room makes the build run again)
                    seen_cap = min(N, int(self.seen_of[k] * max(SEEN_MARGIN, 1.0)) + 4096)
                    seen = torch.empty(max(seen_cap, 1), dtype=torch.int32, device=dev)
                    seen_n = stats[li, 4:5]
                    # the positions whose level li - 1 context occurred: the bits its ng_pos_summary set
                    elib.cub("ng_bits_list32", hit_bits, hit_bits.numel(), seen, seen_cap, seen_n, None)
                else:
                    seen = torch.nonzero(out[1, li - 1] > 0).squeeze(1).to(torch.int32)
                    self.seen_of[k] = int(seen.numel())
            kept = k in keep
            ktop = 8 if (kept or cnt_top is not None) else _record_width(topk)
            q0, q1 = self._event("qindex", k, N)
            q0.record()
            vi = QueryIndex(elib, x, avail, k, seen, expect=self.contexts_of.get(k), defer=_defer, n_dev=seen_n,
                            counters=stats[li, 5:8], load=self._load(k, prev, ktop, cnt_top))
            q1.record()
            if vi.n is None:
                pending.append((li, k))
            else:
                self.contexts_of[k] = vi.n
            t1 = time.perf_counter()
            ev_fn = lambda name, n, k=k: self._event(name, k, n)  # noqa: E731
            _, W = w_bits(vi.ids)
            use32 = cnt_top is None and W <= W_MAX and k not in self.wide
            if not use32 and seen_n is not None:  # the 64-bit count takes an exact list: read its length
                seen = seen[: int(seen_n.item())]
                seen_n = None
            mbits = self._mbits(W, vi.ids, ktop) if use32 else 0
            seg = self._emit(k, vi, x, bms, regions, R, W if use32 else 0,
                             stats[li, 3:4].view(torch.int32) if use32 else None, mbits)
            t2 = time.perf_counter()
            if use32:
                # the 32-bit count: records made without sorting the pairs, every size read once after the last level
                c = count32(elib, seg, vi.ids, ktop, (vi.ctx_of, tgt, seen, seen_n), self.events_of.get(k),
                            self.dratio.get(k, 1.0), ev_fn, self.min_pbits.get(k, 0), stat=stats[li],
                            mbits=mbits)
                del seg
                checks32.append((k, li, c.pbits, vi.ids, seen_cap if seen_n is not None else -1))
                sm = c
                res.info[k] = dict(contexts=vi.n, ids=vi.ids, pairs=None, events=None, pbits=c.pbits, hits=None)
            else:
                c = count_events(elib, elib, None, 0, vi.ids, self.dratio.get(k, 1.0), (vi.ctx_of, tgt, seen),
                                 event=ev_fn, seg=seg, presort="ctx")
                del seg
                self.events_of[k] = c.n_ev
                self.dratio[k] = c.U / max(1, c.n_ev)
                if not c.cb:
                    raise RuntimeError(f"k={k}: more large counts than the escape table holds")
                try:
                    sm = summarize(elib, elib, c, vi.ids, ktop, False, ev_fn,
                                   deep_min=cnt_top if cnt_top is not None else None, defer=True)
                except RuntimeError as e:
                    raise RuntimeError(f"k={k}: {e}") from None
                if sm.stat is not None:  # checked once after the last level: no host read per level
                    deferred.append((f"k={k}", sm.stat))
                res.info[k] = dict(contexts=vi.n, ids=vi.ids, pairs=c.U, events=c.n_ev, pbits=c.pbits, hits=None)
            t3 = time.perf_counter()
            thr = None
            if cnt_top is not None and sm.deep.numel():
                thr = elib.zeros(vi.ids, torch.int64, dev)
                e0, e1 = self._event("ctx_kth", k, int(sm.deep.numel()))
                e0.record()
                elib("ng_ctx_kth", sm.words, i32(c.cb), c.esc[0], c.esc[1], u64(partcount.ESC_CAP), sm.rec, sm.deep,
                     sm.deep.numel(), i32(cnt_top), thr)
                e1.record()
            e0, e1 = self._event("pos_gather", k, N)
            e0.record()
            elib("ng_pos_summary", vi.ctx_of, N, 0, vi.ids, tgt, sm.rec, sm.dist, thr, c.qcnt, i32(ktop), i32(topk),
                 i32(li), out[0, li], out[1, li], out[2, li], res.top_tok[li] if topk else None,
                 res.top_cnt[li] if topk else None, res.mask, hit_bits if li + 1 < len(self.levels) else None)
            e1.record()
            if kept:
                res.kept[k] = (vi.ctx_of, sm.rec)
            self.host_s["index"] += t1 - t0
            self.host_s["scan"] += t2 - t1
            self.host_s["count"] += t3 - t2
            del vi, c, sm, thr, seen
        del regions
        host = stats.cpu().tolist() if (checks32 or pending) else None  # the build's one host read
        if checks32 and self._check32(checks32, host, res):
            self.reruns += 1
            return self.build(x, tgt, avail, topk=topk, cnt_top=cnt_top, keep=keep, with_mask=with_mask,
                              stats=want_stats, _defer=_defer)
        if pending:
            checked = QueryIndex.check([(k, None) for _, k in pending], [host[li][5:8] for li, _ in pending])
            redo = False
            for (_, k), (n_ctx, ok) in zip(pending, checked):
                self.contexts_of[k] = n_ctx  # the next build's tables are sized from these
                res.info[k]["contexts"] = n_ctx
                redo |= not ok
            del pending, checked
            if redo:  # an insert found no slot in a table sized from the last build: once more, each level checked
                self.reruns += 1
                return self.build(x, tgt, avail, topk=topk, cnt_top=cnt_top, keep=keep, with_mask=with_mask,
                                  stats=want_stats, _defer=False)
        check_summary(deferred)
        if want_stats:
            for li, k in enumerate(self.levels):
                h = int(self._popcount(bms[k]))
                res.info[k]["hits"] = h
                m = self.level_shards[k]
                self.density[k] = h / max(1, sum(self.sizes[:m]))
                # the positions the level's scan probed: every position of its shards for the first level, else the
                # previous level's hits that pass the gate (the prefix rule included) within its shards
                probed = sum(self.sizes[:m])
                if li and m > self.level_shards[self.levels[li - 1]]:
                    probed = None  # some of its shards are gated by an earlier level's hits: not counted here
                elif li and m:
                    end = (self.starts[m - 1] + self.sizes[m - 1] + 31) // 32
                    n = torch.zeros(1, dtype=torch.int64, device=dev)
                    elib("ng_gate_popcount", bms[self.levels[li - 1]], end, self._pre, n)
                    probed = int(n.item())
                res.info[k]["probed"] = probed
        return res

    def _check32(self, checks: list, host: list, res: LevelOutputs) -> bool:
        """The 32-bit counts' device results (`host`: the build's stats read in one copy): each level's events and
        distinct pairs (kept to size
        the next build), raising on an overflowed emit region, 2^32 or more events, or a total past uint32. Returns
        whether the build must be redone: a level's query positions listed on the device outran their room (the
        levels after it counted from a cut list, so their results are not kept), a partition overfull (counted
        again with one more partition bit) or the escape table full (the level goes to the 64-bit count)."""
        redo = False
        for k, li, pbits, ids, seen_cap in checks:
            n_ev, n_u, fl, scan, n_seen = host[li][:5]
            sfl, n_false = scan & 0xFFFFFFFF, (scan >> 32) & 0xFFFFFFFF
            if seen_cap >= 0:  # the level's query positions were listed on the device
                self.seen_of[k] = max(n_seen, 1)
                if n_seen > seen_cap:  # more than their room: the build runs again with room for them
                    return True
            fl &= 0xFFFFFFFF
            if sfl & 4:
                raise RuntimeError(f"k={k}: an emit region overflowed")
            if n_ev >= 1 << 32:
                raise RuntimeError(f"k={k}: {n_ev} events: the region scatter's offsets are 32-bit")
            if fl & 4:
                raise RuntimeError(f"k={k}: a total does not fit uint32")
            self.events_of[k] = n_ev
            self.dratio[k] = n_u / max(1, n_ev)  # n_u counts an overfull partition's pairs only up to its limit
            if fl & 1:  # a partition held more distinct pairs than its LDS table takes: one more bit, or the 64-bit
                redo = True  # count when there is none
                if pbits >= partcount.pbits32_max(ids):
                    self.wide.add(k)
                else:
                    self.min_pbits[k] = pbits + 1
            if fl & 2:
                self.wide.add(k)
                redo = True
            res.info[k].update(pairs=n_u, events=n_ev, false_hash_hits=n_false)
        return redo

    def _popcount(self, bm: torch.Tensor) -> int:
        n = torch.zeros(1, dtype=torch.int64, device=bm.device)
        self.elib("popcount", bm, bm.numel(), n)
        return int(n.item())

    def _mode(self, si: int, scanned: list) -> int:
        """A shard's si-th scanned level's scan: a lane per position (0) for the first level and behind a dense
        previous level, the LDS-listed set positions (2) behind a sparser one, or below LIST_DENSITY the set positions
        listed in memory first (3). Densities are the last build's (dense when unknown)."""
        if si == 0:
            return 0
        d = self.density.get(scanned[si - 1])
        if d is None or d >= 0.5:
            return 0
        return 3 if d < LIST_DENSITY else 2

    def _load(self, k: int, prev, ktop: int, cnt_top) -> float | None:
        """Level k's query-table load: DENSE_LOAD where its scan probes every position (the first level, or behind a
        dense one) and a table at that load keeps the count's layout of one at the default load (the 32-bit count, its
        runs mode: the same at both sizes, from the last build's context count); else None (the default)."""
        expect = self.contexts_of.get(k)
        if expect is None or (prev is not None and self._mode(1, [prev, k]) != 0):
            return None

        def layout(load: float) -> tuple:
            ids = int(max(expect, 1) * max(EXPECT_MARGIN, 1.0) / load) + 1024 + QTAIL
            return w_bits(ids)[1] <= W_MAX, partcount.runs_fit(ids, ktop)

        use32 = cnt_top is None and k not in self.wide
        return DENSE_LOAD if use32 and layout(DENSE_LOAD) == layout(QLOAD) else None

    @staticmethod
    def _mbits(W: int, ids: int, ktop: int) -> int:
        """The 32-bit count's event key bits mixed: those below the first digit (events keyed by context range, the
        count's runs mode) where the runs mode fits the level, else all W."""
        return key_mbits(W) if partcount.runs_fit(ids, ktop) else W

    def _emit(self, k, vi, x, bms, regions, R, wbits=0, flags=None, mbits=0):
        """Level k's scan of every shard it counts, hits emitted to per-block regions with each block's top-digit
        histogram: count_events' seg = (regions, R, ev_count, dhist, nseg, flags). wbits: events kmix(pair key,
        wbits, mbits) (part.h; mbits 0: wbits) with histograms of their first_digit(wbits) top bits (count32's), else
        mix64(pair key). flags: the
        scan's two int32 flags (zeroed; e.g. a view into the build's stats), else new."""
        elib, dev, G = self.elib, self.tok.device, self.grid
        shards = [i for i in range(len(self.sizes)) if i < self.level_shards[k]]
        nseg = len(shards) * G
        # every scan block writes its event count (an empty shard's scan writes zeros)
        ev_count = torch.empty(nseg, dtype=torch.int32, device=dev) if nseg else elib.zeros(1, torch.int32, dev)
        last = self.events_of.get(k)
        dbits = first_digit(wbits) if wbits else 8
        dhist = torch.empty((1 << dbits) * max(nseg, 1), dtype=torch.int32, device=dev) \
            if wbits or last is None or last >= partcount.SEG_MIN_EVENTS * nseg else None
        if flags is None:
            flags = elib.zeros(2, torch.int32, dev)
        scans = {tuple(q for q in self.levels if i < self.level_shards[q]) for i in shards}
        if len(shards) > 1 and len(scans) == 1:
            # every shard scans the same levels: one launch over all of them (the SENT gaps between shards hold no
            # context), unless this is the first level and shards may still be arriving (each waits for its copy)
            scanned = list(scans.pop())
            si = scanned.index(k)
            if si > 0 or self.ready is None:
                return self._emit_all(k, vi, x, None if si == 0 else bms[scanned[si - 1]], bms[k], shards, regions,
                                      flags, self._mode(si, scanned), wbits, mbits)
        for j, i in enumerate(shards):
            st, n = self.starts[i], self.sizes[i]
            n32 = (n + 31) // 32 * 32
            self._wait(i)
            scanned = [q for q in self.levels if i < self.level_shards[q]]
            si = scanned.index(k)
            bm_in = None if si == 0 else bms[scanned[si - 1]][st // 32 :]
            mode = self._mode(si, scanned)
            if mode == 3:
                if self._plist is None or self._plist.numel() < n32:
                    self._plist = torch.empty(max(self.sizes) + 64, dtype=torch.int64, device=dev)
                if k != self._no_bm:
                    elib.fill(bms[k][st // 32 : (st + n32) // 32], 0)  # the list scan only sets its hits' bits
                n_list = elib.zeros(1, torch.int64, dev)
                b0, b1 = self._event("bits_list", k, n32)
                b0.record()
                elib.cub("ng_bits_list", bm_in, n32 // 32, self._plist, n_list, self._pre)
                b1.record()
            e0, e1 = self._event("scan_emit", k, n32, mode)
            e0.record()
            dh = dhist[j * G :] if dhist is not None else None
            if mode == 3:
                elib("ng_scan_emit_list", self.tok[st:], self._plist, n_list, i32(k), vi.table, u64(vi.cap), vi.rep,
                     x, bms[k][st // 32 :] if k != self._no_bm else None, regions[j * G * R :], u64(R),
                     ev_count[j * G :], flags, i32(G), dh, nseg, i32(wbits), i32(dbits), i32(mbits))
            else:
                elib("ng_scan_emit", self.tok[st:], n32, i32(k), bm_in, bms[k][st // 32 :], vi.table, u64(vi.cap),
                     vi.rep, x, regions[j * G * R :], u64(R), ev_count[j * G :], flags, i32(G), i32(mode), dh, nseg,
                     self._pre, i32(wbits), i32(dbits), i32(mbits))
            e1.record()
        return regions, R, ev_count, dhist, nseg, flags  # count_events checks the flags with its first read

    def _emit_all(self, k, vi, x, bm_in, bm_out, shards, regions, flags, mode, wbits=0, mbits=0):
        """_emit of a level whose shards all scan the same levels, in one launch from the first shard's start to the
        last one's end: a lane per position (mode 0), the LDS-listed set positions (2), or one list of the previous
        level's set bits and one list scan (3); events as _emit's by wbits."""
        elib, dev, G = self.elib, self.tok.device, self.grid
        lo = self.starts[shards[0]]
        hi = self.starts[shards[-1]] + (self.sizes[shards[-1]] + 31) // 32 * 32
        for i in shards:
            self._wait(i)
        n = hi - lo
        R = -(-max(n, 1) // (G * 256)) * 256 if mode == 3 else emit_region(n, G)
        if G * R > regions.numel():
            raise RuntimeError(f"k={k}: the emit regions are too small for one scan over every shard")
        ev_count = torch.empty(G, dtype=torch.int32, device=dev)  # every scan block writes its event count
        last = self.events_of.get(k)
        dbits = first_digit(wbits) if wbits else 8
        dhist = torch.empty((1 << dbits) * G, dtype=torch.int32, device=dev) \
            if wbits or last is None or last >= partcount.SEG_MIN_EVENTS * G else None
        if mode == 3:
            if self._plist is None or self._plist.numel() < n:
                self._plist = torch.empty(n + 64, dtype=torch.int64, device=dev)
            if k != self._no_bm:
                elib.fill(bm_out[lo // 32 : hi // 32], 0)  # the list scan only sets its hits' bits
            n_list = elib.zeros(1, torch.int64, dev)
            b0, b1 = self._event("bits_list", k, n)
            b0.record()
            elib.cub("ng_bits_list", bm_in[lo // 32 :], n // 32, self._plist, n_list, self._pre)
            b1.record()
        e0, e1 = self._event("scan_emit", k, n, mode)
        e0.record()
        if mode == 3:
            elib("ng_scan_emit_list", self.tok[lo:], self._plist, n_list, i32(k), vi.table, u64(vi.cap), vi.rep, x,
                 bm_out[lo // 32 :] if k != self._no_bm else None, regions, u64(R), ev_count, flags, i32(G), dhist, G,
                 i32(wbits), i32(dbits), i32(mbits))
        else:
            elib("ng_scan_emit", self.tok[lo:], n, i32(k), None if bm_in is None else bm_in[lo // 32 :],
                 bm_out[lo // 32 :], vi.table, u64(vi.cap), vi.rep, x, regions, u64(R), ev_count, flags, i32(G),
                 i32(mode), dhist, G, self._pre, i32(wbits), i32(dbits), i32(mbits))
        e1.record()
        return regions, R, ev_count, dhist, G, flags
