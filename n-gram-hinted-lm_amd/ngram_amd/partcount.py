"""Counting (context id, next token) events without global atomics, shared by CountBuild's "part" mode and the
longest match's counting phase (libngram_amd.so's partitioned-count entry points; no counterpart in the reference,
whose counts go through one atomic hash table per level, record_367_gpu_counts/track_1_short/counts/kernels.cu:132-247).

An emitting scan (ng_scan_emit) leaves each block's events — mix64(context id << 16 | next), a bijection of the pair
key — in the block's own region. `pack_events` packs the regions into one array; `count_events` sorts the events by
their top pbits (a hash partition of the pairs, sized so a partition holds about PART_TARGET distinct pairs: the LDS
table holds 7000), counts every partition in LDS (ng_part_count), answers the lookups (the query positions' (context,
target) pairs, hashed and sorted the same way) and packs the distinct pairs, by default as one word each: pair key <<
(48 - cb) | count (a count too large for the field also goes to an escape table). `summarize` sorts the words by
context (keys only) and makes each present context's record: total, pairs, top entries (ng_ctx_summary), which
ng_pos_summary gathers per query position.

On MI355X, global atomics run at about 27 G/s on scattered slots and 80 M/s on one address (a hot pair's chain);
here every event is counted by an LDS atomic and moved by coalesced streams."""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from .lib import Lib, i32, u64

PART_TARGET = 4096  # distinct pairs per partition aimed at (the LDS table takes up to 7000)
PART_BLOCKS = 2048  # count blocks, each a run of consecutive partitions
PART_MIN_BITS = 11  # at least this many partition bits: enough blocks for the lookups as well
ESC_CAP = 1 << 20  # packed pairs whose count exceeds the word's count field, per level
PACK_MIN_BITS = 0  # context-id bits of the packed words at least this (up to 44: a narrower count field)
SEG_MIN_EVENTS = 4096  # events per scan region from which the partition sort's first pass reads the regions directly


def emit_region(L: int, grid: int) -> int:
    """The per-block region an emitting scan of L positions with `grid` blocks needs (ng_emit_region)."""
    per = grid * 8192
    return -(-L // per) * 8192


def _no_event(name: str, n: int):
    class _E:
        def record(self):
            pass

    return _E(), _E()


class _HostRead:
    """A small device tensor copied to pinned host memory without a wait: the launches enqueued after it keep the GPU
    busy while the host waits for this copy alone (get), instead of the GPU idling until the host's next launch."""

    def __init__(self, t: torch.Tensor):
        self.host = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
        self.host.copy_(t, non_blocking=True)
        self.ready = torch.cuda.Event()
        self.ready.record()

    def get(self) -> list:
        self.ready.synchronize()
        return self.host.tolist()


def pack_events(elib: Lib, regions: torch.Tensor, R: int, ev_count: torch.Tensor, nseg: int, event=_no_event):
    """The regions' events (segment s = ev_count[s] items at s * R) packed into one array: (events, n)."""
    dev = regions.device
    offs = torch.empty(nseg + 1, dtype=torch.int64, device=dev)
    elib("ng_seg_offsets", ev_count, nseg, offs)
    n_ev = int(offs[nseg].item())
    ev = torch.empty(max(n_ev, 1), dtype=torch.int64, device=dev)
    e0, e1 = event("gather", n_ev)
    e0.record()
    elib("ng_seg_gather", regions, None, u64(R), None, ev_count, nseg, offs, ev, None)
    e1.record()
    return ev, n_ev


@dataclass
class Counted:
    """A level's distinct pairs: `pairs` (U packed words when cb > 0, else pair keys with `counts`), the escape table
    `esc` (keys, counts) of packed words, per-lookup target counts `qcnt`, the partition bits used, the events."""

    pairs: torch.Tensor
    counts: torch.Tensor | None
    esc: tuple | None
    qcnt: torch.Tensor | None
    U: int
    pbits: int
    cb: int
    n_ev: int = 0
    presorted: int = -1  # packed words already grouped by their presort_bits-bit digit at bit presorted (-1: not)
    presort_bits: int = 0


def presort_bits(total: int) -> int:
    """The width (8 to 11) of a sort's first digit over `total` bits that leaves the fewest 8-bit passes after it."""
    return min(range(8, 12), key=lambda w: (-(-max(total - w, 0) // 8), w))


def count_events(elib: Lib, lib: Lib, ev: torch.Tensor | None, n_ev: int, n_ids: int, ratio: float = 1.0,
                 lookups: tuple | None = None, packed: bool = True, event=_no_event, seg: tuple | None = None,
                 presort: str | None = None) -> Counted:
    """Count n_ev events of context ids below n_ids. `ratio`: distinct pairs per event expected (sizes the
    partitions; a partition found too full repeats the count with one more bit). `lookups` (ctx_of int32 [N], tgt
    int16 [N], positions int32 or None): qcnt[i] = the count of (ctx_of[i], tgt[i]) for the listed positions (all
    without a list), 0 where absent, out of range or not listed. `packed`: pairs as packed words (falls back to keys +
    counts when the escape table overflows). `seg` (regions, R, ev_count, dhist, nseg[, flags]): the events straight
    from an emitting scan's regions with its digit histograms (ng_scan_emit's dhist, digit-major with stride nseg;
    None: the regions are packed) and, if given, the scan's flags (raises on a region overflow, bit 4, before any
    region is read); ev and n_ev are then unused: the first partition pass reads the regions (ng_seg_scatter) and groups by the top 8 bits,
    the later passes sort the bits below them. `presort` ("ctx" / "pair", packed words only): the words come out
    already through the first pass of summarize's sort (by context / by pair key), read from the count's outputs."""
    msd = 0
    emit_flags = seg[5] if seg is not None and len(seg) > 5 else None
    if seg is not None and seg[3] is None:  # no digit histograms: the regions are packed
        regions, R, ev_count, _, nseg = seg[:5]
        if emit_flags is not None and int(emit_flags[0].item()) & 4:
            raise RuntimeError("an emit region overflowed")
        ev, n_ev = pack_events(elib, regions, R, ev_count, nseg, event)
    elif seg is not None:
        regions, R, ev_count, dhist, nseg = seg[:5]
        dev = regions.device
        dpre = torch.empty(max(256 * nseg, 1), dtype=torch.int32, device=dev)
        small = torch.zeros(2, dtype=torch.int64, device=dev)  # [the events, the scan's flags]: one copy
        elib.cub("ng_exclusive_scan_u32", dhist, dpre, 256 * nseg, small[:1])
        if emit_flags is not None:
            small[1:].copy_(emit_flags[:1])
        read = _HostRead(small)
        # the first partition pass, launched before the host reads the total so that the GPU works while the host
        # waits: its output holds every region's capacity and the scatter drops anything placed beyond it, so an
        # overflowed region or a wrapped total, raised below, writes nothing out of bounds
        cap = nseg * R
        ev = torch.empty(max(cap, 1), dtype=torch.int64, device=dev)
        e0, e1 = event("partition", cap)
        e0.record()
        elib("ng_seg_scatter", regions, u64(R), None, ev_count, dpre, nseg, i32(56), i32(8), ev, u64(cap))
        e1.record()
        msd = 1
        n_ev, fl = read.get()
        if fl & 4:
            raise RuntimeError("an emit region overflowed")
        if n_ev >= 1 << 32:
            raise RuntimeError(f"{n_ev} events: the region scatter's offsets are 32-bit")
        del dpre
    dev = ev.device
    cb = max(1, (max(n_ids, 2) - 1).bit_length(), PACK_MIN_BITS) if packed else 0
    N = nq = 0
    if lookups is not None:
        ctx_of, tgt, qpos = lookups
        N = ctx_of.numel()
        nq = N if qpos is None else qpos.numel()
        qk = torch.empty(max(nq, 1), dtype=torch.int64, device=dev)
        qv = torch.empty(max(nq, 1), dtype=torch.int32, device=dev)
        e0, e1 = event("partition", nq)
        e0.record()
        elib("ng_part_lookups", ctx_of, tgt, qpos, nq, 0, n_ids, qk, qv)
        e1.record()
    min_bits = min(PART_MIN_BITS, 24) if N else 0  # lookups want enough partitions (blocks) to spread over
    pbits = max(min_bits, min(24, math.ceil(math.log2(max(1.0, n_ev * ratio / PART_TARGET)))))

    def sort_by_partition(k_in, v_in, n):
        """Keys (and values) in the partition order of msd / pbits."""
        k_out = torch.empty(max(n, 1), dtype=torch.int64, device=dev)
        v_out = torch.empty(max(n, 1), dtype=torch.int32, device=dev) if v_in is not None else None
        if not n:
            return k_out, v_out
        if not msd:
            lib.cub("sort_pairs", k_in, k_out, v_in, v_out, n, i32(64 - pbits), i32(64))
        elif pbits > 8:
            lib.cub("sort_pairs", k_in, k_out, v_in, v_out, n, i32(64 - pbits), i32(56))
        else:
            k_out.copy_(k_in[:n])
            if v_in is not None:
                v_out.copy_(v_in[:n])
        return k_out, v_out

    while True:
        P = 1 << pbits
        start = torch.empty(P + 1, dtype=torch.int64, device=dev)
        qstart = torch.zeros(P + 1, dtype=torch.int64, device=dev)
        sqk = sqv = None
        e0, e1 = event("partition", n_ev)
        e0.record()
        if msd and pbits <= 8:
            sev = ev  # the first pass's grouping by the top 8 bits is already by the top pbits
        else:
            sev, _ = sort_by_partition(ev, None, n_ev)
        elib("ng_part_bounds", sev, n_ev, i32(pbits), i32(msd), start)
        if nq:
            if msd:  # the lookups take the events' two-step order: the top 8 bits, then (stably) the bits below
                qk8 = torch.empty(nq, dtype=torch.int64, device=dev)
                qv8 = torch.empty(nq, dtype=torch.int32, device=dev)
                lib.cub("sort_pairs", qk, qk8, qv, qv8, nq, i32(56), i32(64))
                sqk, sqv = sort_by_partition(qk8, qv8, nq) if pbits > 8 else (qk8, qv8)
                del qk8, qv8
            else:
                sqk, sqv = sort_by_partition(qk, qv, nq)
            elib("ng_part_bounds", sqk, nq, i32(pbits), i32(msd), qstart)
        e1.record()
        G2 = min(P, PART_BLOCKS)
        out_k = torch.empty(max(n_ev, 1), dtype=torch.int64, device=dev)
        out_c = None if cb else torch.empty(max(n_ev, 1), dtype=torch.int32, device=dev)
        esc_k = torch.full((ESC_CAP,), -1, dtype=torch.int64, device=dev) if cb else None
        esc_c = torch.empty(ESC_CAP, dtype=torch.int32, device=dev) if cb else None
        seg_cnt = torch.empty(G2, dtype=torch.int32, device=dev)
        seg_base = torch.empty(G2, dtype=torch.int64, device=dev)
        qcnt = torch.zeros(max(N, 1), dtype=torch.int32, device=dev) if N else None
        small = torch.zeros(2, dtype=torch.int64, device=dev)  # [the distinct pairs counted, the count's flags]
        flags = small[1:].view(torch.int32)[:1]
        dshift = dbits = -1
        if presort and cb:  # the lowest digit of the words' sort range, as wide as saves summarize a radix pass
            dshift = 64 - cb - (16 if presort == "pair" else 0)
            dbits = min(presort_bits(64 - dshift), 64 - dshift)
        dhist = torch.empty((1 << max(dbits, 0)) * G2, dtype=torch.int32, device=dev) if dshift >= 0 else None
        e0, e1 = event("count", n_ev)
        e0.record()
        elib("ng_part_count", sev, start, i32(pbits), sqk, sqv, qstart, out_k, out_c, i32(cb), esc_k, esc_c,
             u64(ESC_CAP if cb else 0), seg_cnt, seg_base, qcnt, dhist, i32(max(dshift, 0)), i32(max(dbits, 1)),
             flags, i32(G2))
        e1.record()
        del sev, sqk, sqv, start, qstart
        # the pairs' offsets computed before the flags are read (and dropped if the count repeats): one copy returns
        # both
        if dhist is not None:  # the words scattered by their lowest sort digit: summarize's first radix pass
            nb = (1 << dbits) * G2
            dpre = torch.empty(nb, dtype=torch.int32, device=dev)
            elib.cub("ng_exclusive_scan_u32", dhist, dpre, nb, small[:1])
        else:
            offs = torch.empty(G2 + 1, dtype=torch.int64, device=dev)
            elib("ng_seg_offsets", seg_cnt, G2, offs)
            small[:1].copy_(offs[G2:])
        read = _HostRead(small)
        # the distinct pairs packed before the host reads how many there are (the GPU works while the host waits),
        # into room for every event, which bounds them; dropped if the count repeats
        pairs = torch.empty(max(n_ev, 1), dtype=torch.int64, device=dev)
        counts = None if cb else torch.empty(max(n_ev, 1), dtype=torch.int32, device=dev)
        if dhist is not None:
            e0, e1 = event("sort", n_ev)
            e0.record()
            elib("ng_seg_scatter", out_k, u64(0), seg_base, seg_cnt, dpre, G2, i32(dshift), i32(dbits), pairs,
                 u64(pairs.numel()))
            e1.record()
        else:
            e0, e1 = event("count", n_ev)
            e0.record()
            elib("ng_seg_gather", out_k, out_c, u64(0), seg_base, seg_cnt, G2, offs, pairs, counts)
            e1.record()
        U, fl = read.get()
        fl &= 0xFFFFFFFF
        if fl & 2:  # more large counts than the escape table holds: count again, unpacked
            cb = 0
            continue
        if not fl & 1:
            break
        if pbits >= 24:
            raise RuntimeError("a partition holds too many distinct pairs at 24 bits")
        pbits += 1
    del ev
    return Counted(pairs, counts, (esc_k, esc_c) if cb else None, qcnt, U, pbits, cb, n_ev, dshift,
                   dbits if dhist is not None else 0)


RECORD_WORDS = {1: 4, 2: 8, 4: 8, 8: 16}  # u32 words of a context record for top 1, 2, 4, 8

P32_SLOTS = 14336  # slots of the 32-bit count's per-partition table (pairs32.h), the size of a partition's slab
P32_TARGET = 6144  # distinct pairs per partition aimed at by the 32-bit count (its LDS table takes up to 11000)
P32_LIMIT = 11000  # distinct pairs at which the 32-bit count declares a partition overfull (at most 11000)
PACK32_MIN_BITS = 0  # context bits of the 32-bit count's packed words at least this (a narrower count field)
WORD_DIGIT = 8  # the 32-bit count's words are grouped by context first by this many top id bits (at least)
AGG_ID_BITS = 11  # context ids per group of words whose records ng_ctx_agg makes in one block: at most 2^11 (2^10 for
                  # top 8, whose LDS then lets two blocks share a compute unit)
W_MAX = 42  # the widest pair key (context-id bits + 16) the 32-bit count narrows in its first pass: that pass's digit
            # is at most 10 bits (the emitting scan's histogram) and must leave at most 32 bits below it
W_WIDE = 47  # the widest it takes at all (wider ones are narrowed by the second pass; context ids below 2^31)


def w_bits(n_ids: int) -> tuple[int, int]:
    """(cb, W) of a level with n_ids context ids: the context-id bits and the pair-key bits W = cb + 16."""
    cb = max(1, (max(n_ids, 2) - 1).bit_length())
    return cb, cb + 16


def first_digit(W: int) -> int:
    """The 32-bit count's first-pass digit width for W-bit pair keys: at least 8, and at most 32 bits below it (at most
    10 bits: wider keys keep 64 bits through the first pass)."""
    return min(max(8, W - 32), 10)


def key_mbits(W: int) -> int:
    """The bits of a W-bit pair key that its 32-bit count event mixes (kmix, part.h) where the event is keyed by context
    range: those below the first pass's digit, which then holds the top context-id bits (so a first-pass bucket is a
    range of context ids, and its partitions hold the pairs of those contexts only: count32's runs mode)."""
    return W - first_digit(W)


@dataclass
class Counted32:
    """A level counted by count32: per context id its record (int32 [n_ids, RECORD_WORDS[ktop]]) and pair count
    dist (int32 [n_ids], 0 for absent contexts), per query position the target's count qcnt (int32 [N]), and the
    device-side results the host checks once per build (`stat`: int64 [8] = events, distinct pairs, the count's flags,
    the scan's flags as two int32 (its bits; its false hash hits, hashed keys of k > 4 found in the query table whose
    tokens differ) where the caller's scan wrote them there, then the caller's own; bit 0 of the count's flags: a
    partition overfull, bit 1: the escape table full, bit 2: a total reached 2^32; bit 2 of the scan's: a region
    overflowed)."""

    rec: torch.Tensor
    dist: torch.Tensor | None
    qcnt: torch.Tensor | None
    stat: torch.Tensor
    pbits: int
    cb: int
    esc: tuple
    W: int = 0
    slab: torch.Tensor | None = None  # with slabs: the count's per-partition tables (pairs32.h), [2^pbits * 14336]
    words: torch.Tensor | None = None  # with deep_min: the words grouped by context (ng_ctx_agg's input) ...
    wstart: torch.Tensor | None = None  # ... their groups' starts (groups of 2^ibits ids)
    ibits: int = 0
    deep: torch.Tensor | None = None  # with deep_min: the contexts of more than deep_min pairs (the first deep_n)
    deep_n: torch.Tensor | None = None  # int64 [2] on the device: the deep contexts, the present contexts


def pbits32_max(n_ids: int) -> int:
    """The most partition bits the 32-bit count takes for a level of n_ids context ids."""
    W = w_bits(n_ids)[1]
    return min(first_digit(W) + 11, W - 1)


def count32(elib: Lib, seg: tuple, n_ids: int, ktop: int, lookups: tuple | None, n_events: int | None,
            ratio: float = 1.0, event=_no_event, min_pbits: int = 0, slabs: bool = False,
            deep_min: int | None = None, with_dist: bool = True, agg_grid: int = 0,
            stat: torch.Tensor | None = None, mbits: int | None = None) -> Counted32:
    """Count a level's events emitted by ng_scan_emit in the W-bit mode (wbits = W = w_bits(n_ids)[1], dbits =
    first_digit(W); seg = (regions, R, ev_count, dhist, nseg, scan flags)) and make every present context's record
    (top ktop) without a host read: the passes and the count of pairs32.hip. `n_events`: the level's events (the last
    build's; None: read from the device here, one host sync), which with `ratio` (distinct pairs per event) sizes the
    partitions, with at least min_pbits partition bits (and at most pbits32_max(n_ids)); `lookups` as count_events',
    and optionally a fourth entry: a device-side count (int64 [1]) of the listed positions, at most their number.
    Events wider than W_MAX bits (first digit 10 bits, so more than 32 bits below it) keep 64 bits through the first
    pass and are narrowed by the second (ng_msd_pass_narrow). `slabs`: also keep the count's per-partition tables
    (Counted32.slab) for queries after the build; `deep_min`: keep the words grouped by context and list the contexts
    of more than deep_min pairs (for their CNT_TOP thresholds, ng_ctx_kth_grouped). Without with_dist, dist is None
    (the records hold each present context's pairs). agg_grid: ng_ctx_agg's blocks (0: one per group of ids; a couple
    per compute unit for many light groups, each block then walking its groups with the next one's words loaded
    ahead). `stat`: the caller's int64 [>= 8] of zeros for Counted32.stat (e.g. a row of one tensor every level of a
    build shares, read once); its fourth entry holds the scan's two int32 flags where the caller's seg flags are a view
    of it. `mbits`: the events' mixed bits (the scan's; None: W, every bit). With key_mbits(W) (events keyed by context
    range) and without slabs or deep_min, the count leaves each partition's words grouped by context sub-range (runs)
    and the records are made from those runs directly (ng_ctx_agg_runs), without grouping the words by context, as long
    as a bucket has at most 256 partitions and 64 sub-ranges."""
    regions, R, ev_count, dhist, nseg, scan_flags = seg
    dev = regions.device
    idb, W = w_bits(n_ids)
    cb = max(idb, PACK32_MIN_BITS)  # the words' context field: idb bits used, cb - idb zero bits above them
    if W > W_WIDE:
        raise ValueError(f"{n_ids} context ids: wider than the 32-bit count takes")
    d1 = first_digit(W)
    M = W if mbits is None else mbits
    cap = nseg * R
    if stat is None:
        stat = elib.zeros(8, torch.int64, dev)
    # stat: events, distinct pairs, count flags, the scan's flags (two int32: overflow bits, false hash hits) where the
    # caller put them there, the caller's fifth (the level's listed query positions) and beyond
    ev_tot, u_tot = stat[0:1], stat[1:2]
    flags = stat[2:3].view(torch.int32)[:1]
    dpre = torch.empty((1 << d1) * nseg, dtype=torch.int32, device=dev)
    elib.cub("ng_exclusive_scan_u32", dhist, dpre, (1 << d1) * nseg, ev_tot)
    if n_events is None:
        n_events = int(ev_tot.item())
    # events keyed by context range (M < W) fill only the partitions of the used share of the id bits
    used = n_ids / (1 << idb) if M < W else 1.0
    pbits = max(d1 + 1, W - 31, PART_MIN_BITS if lookups is not None else 0, min_pbits,
                math.ceil(math.log2(max(1.0, n_events * ratio / P32_TARGET / used))))
    pbits = min(pbits, pbits32_max(n_ids))
    d2 = pbits - d1
    e0, e1 = event("partition", cap)
    e0.record()
    ev32b = torch.empty(max(cap, 1), dtype=torch.int32, device=dev)
    P = 1 << pbits
    start = torch.empty(P + 1, dtype=torch.int64, device=dev)
    if W <= W_MAX:
        ev1 = torch.empty(max(cap, 1), dtype=torch.int32, device=dev)
        elib("ng_seg_scatter_narrow", regions, u64(R), None, ev_count, dpre, nseg, i32(W - d1), i32(d1), ev1, u64(cap))
        elib.cub("ng_msd_pass", ev1, dpre, nseg, i32(d1), ev_tot, u64(cap), i32(W - pbits), i32(d2), ev32b, start)
    else:  # wide keys: 64 bits through the first pass, narrowed by the second
        ev1 = torch.empty(max(cap, 1), dtype=torch.int64, device=dev)
        elib("ng_seg_scatter", regions, u64(R), None, ev_count, dpre, nseg, i32(W - d1), i32(d1), ev1, u64(cap))
        elib.cub("ng_msd_pass_narrow", ev1, dpre, nseg, i32(d1), ev_tot, u64(cap), i32(W - pbits), i32(d2), ev32b,
                 start)
    del ev1, dpre
    N = nq = 0
    sqk = sqv = None
    if lookups is not None:
        ctx_of, tgt, qpos = lookups[:3]
        qn = lookups[3] if len(lookups) > 3 else None  # a device-side count of qpos's entries
        N = ctx_of.numel()
        nq = N if qpos is None else qpos.numel()
    if nq:
        qk = torch.empty(nq, dtype=torch.int64, device=dev)
        qv = torch.empty(nq, dtype=torch.int32, device=dev)
        elib("ng_part_lookups_w", ctx_of, tgt, qpos, nq, qn, 0, n_ids, i32(W), i32(M), qk, qv)
        sqk = torch.empty(nq, dtype=torch.int64, device=dev)
        sqv = torch.empty(nq, dtype=torch.int32, device=dev)
        elib.cub("sort_pairs", qk, sqk, qv, sqv, nq, i32(64 - pbits), i32(64))
        del qk, qv
        qstart = torch.empty(P + 1, dtype=torch.int64, device=dev)
        elib("ng_part_bounds", sqk, nq, i32(pbits), i32(0), qstart)  # every partition's bound
    else:
        qstart = elib.zeros(P + 1, torch.int64, dev)  # no lookups
    e1.record()
    # the count's blocks: one per compute unit (its LDS table takes a compute unit's LDS), each a run of consecutive
    # partitions of about equal events; more blocks, run in turns, were slower (c3: 2048, 768, 512 and 256 blocks,
    # 12.8, 12.2, 12.0 and 11.7 ms a step; 384, a second round for half the units, 14.8 ms)
    G2 = min(P, torch.cuda.get_device_properties(dev).multi_processor_count)
    agg = AGG_ID_BITS - 1 if ktop >= 8 else AGG_ID_BITS  # top 8: 2^10 ids a group
    # runs mode: a group is a sub-range of 2^ribits ids of a first-pass bucket (2^(idb - d1) ids), run s of each of
    # the bucket's 2^d2 partitions
    ribits = min(agg, idb - d1)
    rgbits = idb - d1 - ribits
    if M == W - d1 and not slabs and deep_min is None and d2 <= 8 and rgbits <= 6:
        return _count32_runs(elib, n_ids, ktop, W, M, cb, d1, d2, pbits, P, cap, ev32b, start, sqk, sqv, qstart, N,
                             ribits, rgbits, G2, flags, stat, with_dist, agg_grid, event)
    # the words' first grouping digit: 8 bits (runs of about 64 words per digit in each 16384-word chunk), more only
    # where the second pass's 11 bits would not reach a group's
    dc = min(idb, max(WORD_DIGIT, idb - agg - 11))
    dtop = 64 - (cb - idb)  # the bit above a word's highest id bit
    out_k = torch.empty(max(cap, 1), dtype=torch.int64, device=dev)
    esc_k = elib.full_ones(ESC_CAP, torch.int64, dev)
    esc_c = torch.empty(ESC_CAP, dtype=torch.int32, device=dev)
    seg_cnt = torch.empty(G2, dtype=torch.int32, device=dev)
    seg_base = torch.empty(G2, dtype=torch.int64, device=dev)
    qcnt = elib.zeros(max(N, 1), torch.int32, dev) if N else None
    dh2 = torch.empty((1 << dc) * G2, dtype=torch.int32, device=dev)
    slab = torch.empty(P * P32_SLOTS, dtype=torch.int64, device=dev) if slabs else None
    e0, e1 = event("count", cap)
    e0.record()
    elib("ng_part_count32", ev32b, start, i32(pbits), i32(W), i32(M), sqk, sqv, qstart, out_k, i32(cb), esc_k, esc_c,
         u64(ESC_CAP), seg_cnt, seg_base, qcnt, dh2, i32(dtop - dc), i32(dc), ctypes.c_uint32(P32_LIMIT), flags,
         i32(G2), slab, None, i32(0), i32(0), i32(0), _live_np(n_ids, W, M, d1, d2), None)
    e1.record()
    del ev32b, start, sqk, sqv, qstart
    # the words grouped by context: by their top dc bits (ng_seg_scatter), then within those groups by the next d2
    # bits (ng_msd_pass64), so that a group holds at most 2^agg ids, whose records ng_ctx_agg makes in LDS
    d2 = max(0, idb - dc - agg)
    ibits = idb - dc - d2
    P2 = 1 << (dc + d2)
    dpre2 = torch.empty((1 << dc) * G2, dtype=torch.int32, device=dev)
    words = torch.empty(max(cap, 1), dtype=torch.int64, device=dev)
    start2 = torch.empty(P2 + 1, dtype=torch.int64, device=dev)
    e0, e1 = event("sort", cap)
    e0.record()
    elib.cub("ng_exclusive_scan_u32", dh2, dpre2, (1 << dc) * G2, u_tot)
    elib("ng_seg_scatter", out_k, u64(0), seg_base, seg_cnt, dpre2, G2, i32(dtop - dc), i32(dc), words, u64(cap))
    if d2:
        elib.cub("ng_msd_pass64", words, dpre2, G2, i32(dc), u_tot, u64(cap), i32(dtop - dc - d2), i32(d2), out_k,
                 start2)
        words, out_k = out_k, words
    else:
        elib.cub("ng_msd_pass64", None, dpre2, G2, i32(dc), u_tot, u64(cap), i32(0), i32(0), None, start2)
    e1.record()
    del out_k, dh2, seg_cnt, seg_base, dpre2
    rec = torch.empty((max(n_ids, 1), RECORD_WORDS[ktop]), dtype=torch.int32, device=dev)
    dist = torch.empty(max(n_ids, 1), dtype=torch.int32, device=dev) if with_dist else None
    deep = deep_n = None
    if deep_min is not None:  # at most (pairs) / (deep_min + 1) contexts have more than deep_min pairs
        deep = torch.empty(cap // (deep_min + 1) + 1, dtype=torch.int64, device=dev)
        deep_n = elib.zeros(2, torch.int64, dev)  # the deep contexts, the present contexts
    e0, e1 = event("ctx_topk", cap)
    e0.record()
    elib("ng_ctx_agg", words, start2, P2, i32(ibits), i32(cb), n_ids, esc_k, esc_c, u64(ESC_CAP), i32(ktop), rec,
         dist, flags, ctypes.c_uint32(deep_min or 0), deep, u64(deep.numel() if deep is not None else 0), deep_n,
         deep_n[1:] if deep_n is not None else None, i32(agg_grid))
    e1.record()
    keep = deep_min is not None
    return Counted32(rec, dist, qcnt, stat, pbits, cb, (esc_k, esc_c), W, slab, words if keep else None,
                     start2 if keep else None, ibits, deep, deep_n)


def _live_np(n_ids: int, W: int, M: int, d1: int, d2: int) -> int:
    """The partitions whose runs and slabs may be read: with events keyed by context range (M < W), those of the
    first-pass buckets holding ids below n_ids (the others hold no events, and the count writes nothing for them);
    else all of them."""
    if M == W:
        return 1 << (d1 + d2)
    return ((max(n_ids, 1) - 1) >> (W - 16 - d1)) + 1 << d2


def runs_fit(n_ids: int, ktop: int) -> bool:
    """Whether count32's runs mode can take a level of n_ids context ids with top-ktop records: a first-pass bucket
    holds at most 64 groups of ids (the count's run digit). The events are then best keyed by context range
    (key_mbits); else by the pair hash over all W bits."""
    idb, W = w_bits(n_ids)
    agg = AGG_ID_BITS - 1 if ktop >= 8 else AGG_ID_BITS
    return idb - first_digit(W) - min(agg, idb - first_digit(W)) <= 6


def _count32_runs(elib: Lib, n_ids, ktop, W, M, cb, d1, d2, pbits, P, cap, ev32b, start, sqk, sqv, qstart, N, ibits,
                  gbits, G2, flags, stat, with_dist, agg_grid, event) -> Counted32:
    """count32's runs mode: the count writes each partition's words grouped by the gbits context-id bits below the
    first pass's digit (gshift = 16 + ibits), and ng_ctx_agg_runs makes the records of each group of 2^ibits ids from
    its runs in the bucket's 2^d2 partitions."""
    dev = ev32b.device
    out_k = torch.empty(max(cap, 1), dtype=torch.int64, device=dev)
    esc_k = elib.full_ones(ESC_CAP, torch.int64, dev)
    esc_c = torch.empty(ESC_CAP, dtype=torch.int32, device=dev)
    seg_cnt = torch.empty(G2, dtype=torch.int32, device=dev)
    seg_base = torch.empty(G2, dtype=torch.int64, device=dev)
    qcnt = elib.zeros(max(N, 1), torch.int32, dev) if N else None
    runs = torch.empty(P << gbits, dtype=torch.int64, device=dev)  # a run's bounds: start | end << 32
    live_np = _live_np(n_ids, W, M, d1, d2)
    e0, e1 = event("count", cap)
    e0.record()
    elib("ng_part_count32", ev32b, start, i32(pbits), i32(W), i32(M), sqk, sqv, qstart, out_k, i32(cb), esc_k, esc_c,
         u64(ESC_CAP), seg_cnt, seg_base, qcnt, None, i32(0), i32(0), ctypes.c_uint32(P32_LIMIT), flags, i32(G2), None,
         runs, i32(gbits), i32(16 + ibits), i32(d2), live_np, stat[1:2])  # stat[1]: the distinct pairs (zero before)
    e1.record()
    del ev32b, start, sqk, sqv, qstart, seg_cnt, seg_base
    rec = torch.empty((max(n_ids, 1), RECORD_WORDS[ktop]), dtype=torch.int32, device=dev)
    dist = torch.empty(max(n_ids, 1), dtype=torch.int32, device=dev) if with_dist else None
    e0, e1 = event("ctx_topk", cap)
    e0.record()
    elib("ng_ctx_agg_runs", out_k, runs, 1 << (d1 + gbits), i32(d2), i32(gbits), i32(ibits), i32(cb), n_ids, esc_k,
         esc_c, u64(ESC_CAP), i32(ktop), rec, dist, flags, None, i32(agg_grid))
    e1.record()
    return Counted32(rec, dist, qcnt, stat, pbits, cb, (esc_k, esc_c), W, None, None, None, ibits, None, None)



@dataclass
class Summary:
    """ng_ctx_summary's outputs: records (int32 [n_ids, RECORD_WORDS[ktop]]), pair counts per context (int32 [n_ids],
    or None), the sorted words, the number of present contexts, the contexts of more than deep_min pairs (int64).
    Deferred (summarize's defer): contexts is -1 and `stat` holds the kernel's statistics and flags for check_summary."""

    rec: torch.Tensor
    dist: torch.Tensor | None
    words: torch.Tensor
    contexts: int
    deep: torch.Tensor | None
    stat: torch.Tensor | None = None


def summarize(elib: Lib, lib: Lib, c: Counted, n_ids: int, ktop: int, zero_records: bool = False, event=_no_event,
              by_pair: bool = False, with_dist: bool = True, deep_min: int | None = None,
              defer: bool = False) -> Summary:
    """Per present context (of packed pairs): its record (total, pairs, the first ktop tokens two per word, their
    counts; for ktop 2 and 8 also its first word's index in the sorted words) and, with_dist, its pair count (0 for
    absent contexts). The words are sorted by context, or with by_pair by pair key. The records of absent contexts are
    zeros only with zero_records. With deep_min: the contexts of more than deep_min pairs. Raises if a total reaches
    2^32. `defer` (without deep_min): no host sync here; the caller passes the Summary to check_summary before it uses
    any output (a host read per level costs the GPU an idle gap)."""
    dev = c.pairs.device
    lo = 64 - c.cb - (16 if by_pair else 0)  # the sort's bit range [lo, 64)
    first = lo + c.presort_bits if c.presorted == lo else lo  # count_events' scatter did the bits below `first`
    if first >= 64:
        sw = c.pairs
    else:
        sw = torch.empty(max(c.U, 1), dtype=torch.int64, device=dev)
        e0, e1 = event("sort", c.U)
        e0.record()
        if c.U:
            lib.cub("sort_pairs", c.pairs, sw, None, None, c.U, i32(first), i32(64))
        e1.record()
    rec = (torch.zeros if zero_records else torch.empty)((n_ids, RECORD_WORDS[ktop]), dtype=torch.int32, device=dev)
    dist = torch.zeros(n_ids, dtype=torch.int32, device=dev) if with_dist else None
    nstat = torch.zeros(258, dtype=torch.int32, device=dev)  # the kernel's statistics, then its flags: one copy
    deep = torch.empty(c.U // (deep_min + 1) + 1, dtype=torch.int64, device=dev) if deep_min is not None else None
    flags = nstat[257:]
    e0, e1 = event("ctx_topk", c.U)
    e0.record()
    elib("ng_ctx_summary", sw, c.U, i32(c.cb), c.esc[0], c.esc[1], u64(ESC_CAP), i32(ktop), rec, dist,
         ctypes.c_uint32(deep_min or 0), deep, nstat, flags)
    e1.record()
    if defer and deep is None:
        return Summary(rec, dist, sw, -1, None, nstat)
    st = nstat.cpu()
    if int(st[257]) & 4:
        raise RuntimeError("a total does not fit uint32")
    if deep is not None:
        deep = deep[: int(st[0])]
    return Summary(rec, dist, sw, int(st[1:257].sum()), deep)


def check_summary(stats: list) -> None:
    """The deferred checks of summarize(defer=True) calls, one host read for all: (name, Summary.stat) pairs; raises
    RuntimeError(f"{name}: a total does not fit uint32") for the first that overflowed."""
    if not stats:
        return
    flags = torch.stack([st[257] for _, st in stats]).cpu().tolist()
    for (name, _), f in zip(stats, flags):
        if f & 4:
            raise RuntimeError(f"{name}: a total does not fit uint32")


def record_tops(rec: torch.Tensor, ktop: int):
    """The top tokens (int16 [n, ktop]) and counts (int32 [n, ktop]) of context records."""
    tokw = (ktop + 1) // 2
    return rec[:, 2 : 2 + tokw].contiguous().view(torch.int16)[:, :ktop], rec[:, 2 + tokw : 2 + tokw + ktop].contiguous()
