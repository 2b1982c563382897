"""Corpus-wide exact count tables on one MI355X behind exact_match's CountTable surface (exact_match/exact_match.pyi
:100-118; exact_match/src/count_table.rs :173-438): `create` (read the shards, before the clock), `build` (on the
clock: every level), `query_counts`, `query_rows`, `sizes`, `release`, `levels`, `tokens`; plus `query_topk` (each
level's top-k next tokens per position, configuration c2) and `query_device` (the same on GPU
tensors, for callers that keep their queries in device memory).

Definitions (count_table.rs:6-9, kgram.rs's): an occurrence of a k-context is any k consecutive tokens within one
shard and the token after them (it may cross a BOS); a query position's k-context is the k tokens ending at it, valid
iff they lie in its segment (segments start at the first query token and at every BOS). Per level and position:
tot (uint32), dist (uint16, at most 65535), cnt (uint32: the count of the position's next token if among its
context's top CNT_TOP = 1024 next tokens by count descending then token ascending, or any rank when top >= 65536);
0 where the context is invalid or never occurred. Keys: packed tokens for k <= 4 (exact), a 64-bit polynomial hash
beyond (count_table.rs:11-14: ~2^-64 per pair of contexts to merge).

GPU layout per level (libngram_amd.so: ng_table_emit32, the 32-bit count of partcount.count32 (pairs32.hip),
ng_ctx_kth_grouped, ng_table_query32, ng_table_lookup, ng_pos_rows): the context table (u64 keys, slot = context id),
the count's per-partition pair tables kept as slabs (2^pbits partitions of the W-bit pair hash wmix(context id << 16
| token, W), W = context-id bits + 16; 14336 u64 slots count << 32 | key each), one 64-byte record per present context
(total, pairs, top 8 tokens and counts) and the CNT_TOP threshold of contexts with more pairs than that. The build
inserts every corpus position's context and appends its event to its block's region (one LDS cursor per block), then
counts the events without global atomics (two grouping passes, an LDS table per partition) and makes the records
from the distinct pairs grouped by context; a query reads its context's record and looks its pair up in the slab of
the pair's partition."""

from __future__ import annotations

import ctypes
import os

import numpy as np
import torch

from .data import BOS, HEADER_BYTES, shard_tokens
from .data import pack_layout as layout
from . import partcount as P
from .lib import Lib, i32, u64

CNT_TOP = 1024
TOPE = 8
COUNTS = (2, 3, 5, 9, 17, 33)
PURITIES = (0.3, 0.5, 0.7, 0.85, 0.95)
EMIT_BLOCKS_PER_CU = 16  # the emitting inserts' blocks (256 threads) per compute unit: their regions are the count's
# first-pass segments, so fewer blocks give longer segments
CTX_MARGIN = 1.25  # a level's context table sized from the last build's contexts holds this many times them at LOAD
LOAD = 0.5  # context-table load factor of the level's bound on contexts (measured: 0.7 and 0.35 are slower)


def _segments_device(x: torch.Tensor, lib: Lib) -> torch.Tensor:
    """avail of query inputs x (int16 tensor): tokens since the segment start, a segment starting at 0 and at BOS."""
    n = x.numel()
    idx = torch.arange(n, device=x.device)
    start = (x.to(torch.int32) & 0xFFFF) == BOS
    start[:1] = True
    seg = torch.empty_like(idx)
    if n:
        lib.cub("inclusive_max", torch.where(start, idx, torch.zeros_like(idx)), seg, n)
    return (idx - seg + 1).to(torch.int32)


class _Level:
    """One built level on the GPU: context table ck (ccap slots), the count's slabs (2^pbits partitions of W-bit pair
    hashes), records rec [ccap, 16] (valid for present contexts), CNT_TOP thresholds thr (None when no context has more
    pairs), the packed words' context bits cb and escape table esc (the records' large counts), counts of contexts and
    pairs."""

    def __init__(self, k, ck, ccap, slab, pbits, W, U, cb, esc, rec, thr, contexts):
        self.k, self.ck, self.ccap = k, ck, ccap
        self.slab, self.pbits, self.W = slab, pbits, W
        self.pairs, self.cb, self.esc = U, cb, esc
        self.rec, self.thr, self.contexts = rec, thr, contexts


class CountTable:
    """Exact next-token counts of every k-context (k of `levels`) in the training shards (count_table.rs), on the GPU:
    create before the clock, build on it, query the validation tokens (inputs + the last target) after it."""

    def __init__(self):
        raise TypeError("use CountTable.create(files, levels, threads, cpus)")

    @staticmethod
    def create(files: list, levels: list[int], threads: int = 1, cpus: list[int] = (), huge_pages: bool = False,
               device=None) -> "CountTable":
        """Before the clock: read the shards `files` (paths; uint16 arrays are also taken) into GPU memory in the
        layout of the scans (SENT gaps). `threads`, `cpus` and `huge_pages` are the CPU build's and have no effect
        here. ValueError on no files, levels not ascending from >= 1, a bad shard or a token above BOS."""
        levels = list(levels)
        if not files or not levels or levels[0] < 1 or any(a >= b for a, b in zip(levels, levels[1:])) or threads < 1:
            raise ValueError(f"need files, ascending levels >= 1 and threads: {levels}")
        self = object.__new__(CountTable)
        self.lib = Lib()
        self._levels = levels
        dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        arrays = []
        for f in files:
            if isinstance(f, (str, bytes, os.PathLike)):
                n = shard_tokens(f)
                arrays.append(np.fromfile(f, dtype="<u2", count=n, offset=HEADER_BYTES))
            else:
                arrays.append(np.ascontiguousarray(f, dtype=np.uint16))
        if any(len(a) and int(a.max()) > BOS for a in arrays):
            raise ValueError("invalid GPT-2 token in the shards")
        self.sizes_ = [len(a) for a in arrays]
        self.starts, self.L = layout(self.sizes_)
        self.tok = torch.full((self.L,), -1, dtype=torch.int16, device=dev)
        for a, st in zip(arrays, self.starts):
            if len(a):
                self.tok[st : st + len(a)].copy_(torch.from_numpy(a.view(np.int16)))
        self._tokens = int(sum(self.sizes_))
        self.tables: list[_Level] = []
        self.built = self.released = False
        self.grid = torch.cuda.get_device_properties(dev).multi_processor_count * EMIT_BLOCKS_PER_CU
        self.events: list = []
        torch.cuda.synchronize(dev)
        return self

    @classmethod
    def from_device(cls, tok: torch.Tensor, sizes: list[int], starts: list[int], levels: list[int],
                    sizing: dict | None = None) -> "CountTable":
        """A table over shards already laid out in GPU memory (`tok` int16 with SENT gaps at layout()'s starts).
        `sizing`: another table's `sizing` (the contexts per occurrence and distinct pairs per event it found per
        level), so that this build sizes its context tables and partitions from them at once; without it the first
        build sizes from the occurrences alone (a table found too small is built again bigger)."""
        self = object.__new__(CountTable)
        if sizing:
            self.ratio = dict(sizing.get("pairs_per_event", {}))
            self.cratio = dict(sizing.get("contexts_per_occurrence", {}))
        self.lib = Lib()
        self._levels = list(levels)
        self.sizes_, self.starts, self.L = list(sizes), list(starts), int(tok.numel())
        self.tok = tok
        self._tokens = int(sum(sizes))
        self.tables, self.built, self.released = [], False, False
        self.grid = torch.cuda.get_device_properties(tok.device).multi_processor_count * EMIT_BLOCKS_PER_CU
        self.events = []
        return self

    @property
    def sizing(self) -> dict:
        """What this table's build found per level, for another table over the same shards (from_device's sizing)."""
        return {"pairs_per_event": dict(getattr(self, "ratio", {})),
                "contexts_per_occurrence": dict(getattr(self, "cratio", {}))}

    @property
    def levels(self) -> list[int]:
        return list(self._levels)

    @property
    def tokens(self) -> int:
        return self._tokens

    def build(self) -> None:
        """On the clock: build every level (once)."""
        if self.built or self.released:
            raise ValueError("the count table is already built")
        self.built = True
        self.reruns = {}
        if not hasattr(self, "ratio"):
            self.ratio = {}
            self.cratio = {}
        for k in self._levels:
            self.tables.append(self._build_level(k))

    def _timed(self, name: str, k: int):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        self.events.append((name, k, e0, e1))
        return e0, e1

    def _build_level(self, k: int) -> _Level:
        lib, dev = self.lib, self.tok.device
        n_k = sum(max(0, n - k) for n in self.sizes_)  # occurrences: an upper bound of contexts, pairs and events
        bound = n_k
        prev = self.tables[-1] if self.tables else None
        if prev is not None and prev.k == k - 1:
            bound = min(bound, prev.pairs)  # a k-context is a (k-1)-context with its next token: one of its pairs
        if k in self.cratio:  # the last build's contexts per occurrence, with a margin (a full table reruns bigger)
            bound = min(bound, int(self.cratio[k] * n_k * CTX_MARGIN) + 1)
        ccap = max(1 << 16, int(bound / LOAD) + 1)
        G = self.grid
        R = -(-max(self.L, 1) // (G * 256)) * 256  # a block's positions at most: its events at most
        reruns = 0
        while True:
            if ccap > 1 << 31:
                raise RuntimeError(f"k={k}: {n_k} occurrences need more than 2^31 context slots")
            _, W = P.w_bits(ccap)
            d1 = P.first_digit(W)
            ck = torch.full((ccap,), -1, dtype=torch.int64, device=dev)
            flags = torch.zeros(2, dtype=torch.int32, device=dev)
            regions = torch.empty(G * R, dtype=torch.int64, device=dev)
            ev_count = torch.empty(G, dtype=torch.int32, device=dev)
            dhist = torch.empty((1 << d1) * G, dtype=torch.int32, device=dev)
            e0, e1 = self._timed("table_emit", k)
            e0.record()
            lib("ng_table_emit32", self.tok, self.L, i32(k), ck, u64(ccap), i32(W), i32(d1), regions, u64(R), ev_count,
                dhist, flags, i32(G))
            e1.record()
            f = int(flags[0].item())
            if f == 0:
                break
            if f & 4:
                raise RuntimeError(f"k={k}: an emit region overflowed")
            reruns += 1
            ccap = min(2 * ccap, 1 << 31)
            del ck, regions
        ev_name = lambda name, n: self._timed(name, k)
        seg = (regions, R, ev_count, dhist, G, flags)
        min_pbits = 0
        while True:
            c = P.count32(lib, seg, ccap, TOPE, None, n_k, self.ratio.get(k, 1.0), ev_name, min_pbits, slabs=True,
                          deep_min=CNT_TOP, with_dist=False, agg_grid=self.grid // EMIT_BLOCKS_PER_CU * 2)
            st = torch.cat([c.stat, c.deep_n]).cpu().tolist()  # one host read: totals, flags, deep contexts
            if int(st[2]) & 1 and c.pbits < P.pbits32_max(ccap):  # a partition overfull: count with a bit more
                min_pbits = c.pbits + 1
                reruns += 1
                continue
            break
        del regions, seg
        if int(st[2]) & 1:
            raise RuntimeError(f"k={k}: a partition holds too many distinct pairs at {c.pbits} bits")
        if int(st[2]) & 2:
            raise RuntimeError(f"k={k}: more large counts than the escape table holds")
        if int(st[2]) & 4:
            raise RuntimeError(f"k={k}: a total does not fit uint32")
        self.reruns[k] = reruns
        ns = c.stat.numel()  # then the deep contexts and the present contexts
        n_ev, U, m, contexts = int(st[0]), int(st[1]), int(st[ns]), int(st[ns + 1])
        self.ratio[k] = max(U, 1) / max(n_ev, 1)
        self.cratio[k] = contexts / max(n_k, 1)
        thr = None
        if m:
            thr = torch.empty(ccap, dtype=torch.int64, device=dev)
            e0, e1 = self._timed("ctx_kth", k)
            e0.record()
            lib("ng_ctx_kth_grouped", c.words, c.wstart, i32(c.ibits), i32(c.cb), c.esc[0], c.esc[1], u64(P.ESC_CAP),
                c.deep, m, None, i32(CNT_TOP), thr)
            e1.record()
        return _Level(k, ck, ccap, c.slab, c.pbits, c.W, U, c.cb, c.esc, c.rec, thr, contexts)

    def _check(self):
        if not self.built or self.released or len(self.tables) != len(self._levels):
            raise ValueError("the count table is not built (or released)")

    @staticmethod
    def _host_tokens(tokens) -> np.ndarray:
        x = np.ascontiguousarray(tokens, dtype=np.uint16)
        if x.ndim != 1 or len(x) < 2 or int(x.max()) > BOS:
            raise ValueError("need 2+ valid tokens")
        return x

    def _slots(self, x: torch.Tensor, avail: torch.Tensor, lv: _Level) -> torch.Tensor:
        n = x.numel()
        keys = torch.empty(n, dtype=torch.int64, device=x.device)
        slot = torch.empty(n, dtype=torch.int32, device=x.device)
        self.lib("val_keys", x, avail, n, i32(lv.k), keys)
        self.lib("ng_table_lookup", keys, n, lv.ck, u64(lv.ccap), slot)
        return slot

    def query_device(self, x: torch.Tensor, tgt: torch.Tensor, avail: torch.Tensor, top: int = CNT_TOP,
                     topk: int = 0) -> dict:
        """Per position and level on the GPU: counts int32 [3, L, n] (tot, dist, cnt; tot and cnt as uint32 bits) and
        with topk > 0 top_tok int16 [L, n, topk] / top_cnt int32 [L, n, topk] (uint16/uint32 bits)."""
        self._check()
        if top != CNT_TOP and top < 1 << 16:
            raise ValueError(f"top must be {CNT_TOP} or at least 65536")
        if not 0 <= topk <= TOPE:
            raise ValueError(f"topk must be in [0, {TOPE}]")
        n, L = x.numel(), len(self.tables)
        out = torch.zeros((3, L, n), dtype=torch.int32, device=x.device)
        res = {"counts": out}
        if topk:
            res["top_tok"] = torch.zeros((L, n, topk), dtype=torch.int16, device=x.device)
            res["top_cnt"] = torch.zeros((L, n, topk), dtype=torch.int32, device=x.device)
        for li, lv in enumerate(self.tables):
            e0, e1 = self._timed("query", lv.k)
            e0.record()
            self.lib("ng_table_query32", x, avail, tgt, n, i32(lv.k), lv.ck, u64(lv.ccap), lv.slab, i32(lv.pbits),
                     i32(lv.W), lv.rec, lv.thr if top == CNT_TOP else None, ctypes.c_uint32(CNT_TOP), i32(topk),
                     out[0, li], out[1, li], out[2, li], res["top_tok"][li] if topk else None,
                     res["top_cnt"][li] if topk else None)
            e1.record()
        return res

    def _device_inputs(self, tokens):
        x = self._host_tokens(tokens)
        dev = self.tok.device
        xt = torch.from_numpy(x.view(np.int16)).to(dev)
        inp, tgt = xt[:-1], xt[1:]
        return inp, tgt, _segments_device(inp, self.lib)

    def query_counts(self, tokens, top: int = CNT_TOP):
        """Per position of `tokens` (the inputs, then the last one's next token) and level: tot (uint32), dist
        (uint16), cnt (uint32), each [n, levels] (count_table.rs query_counts :287-331)."""
        self._check()
        if top != CNT_TOP and top < 1 << 16:
            raise ValueError(f"top must be {CNT_TOP} or at least 65536")
        x, tgt, avail = self._device_inputs(tokens)
        c = self.query_device(x, tgt, avail, top)["counts"]
        tot = c[0].t().contiguous().cpu().numpy().view(np.uint32)
        dist = c[1].t().contiguous().to(torch.int16).cpu().numpy().view(np.uint16)
        cnt = c[2].t().contiguous().cpu().numpy().view(np.uint32)
        return tot, dist, cnt

    def query_topk(self, tokens, k: int = 4):
        """Per position and level its context's k most frequent next tokens (uint16 [n, levels, k], count
        descending then token ascending, 0-padded) and their counts (uint32 [n, levels, k])."""
        self._check()
        x, tgt, avail = self._device_inputs(tokens)
        r = self.query_device(x, tgt, avail, CNT_TOP, k)
        tt = r["top_tok"].permute(1, 0, 2).contiguous().cpu().numpy().view(np.uint16)
        tc = r["top_cnt"].permute(1, 0, 2).contiguous().cpu().numpy().view(np.uint32)
        return tt, tc

    def query_rows(self, tokens, row_levels: list[int], buckets: list[int], entries: int = TOPE):
        """Per position the hint row of the deepest of `row_levels` whose context occurred: cell (int16), its
        `entries` most frequent next tokens (uint16 [n, entries]), weights (uint16: round(count / their sum * 65535),
        ties to even), and its level's index in `buckets` (int8, -1 without a hint) (count_table.rs :338-404)."""
        self._check()
        if not 1 <= entries <= TOPE:
            raise ValueError(f"need 2+ valid tokens and 1 <= entries <= {TOPE}")
        x, tgt, avail = self._device_inputs(tokens)
        use = []
        for k in row_levels:
            if k not in self._levels:
                raise ValueError(f"level {k} is not in the table")
            if k not in buckets:
                raise ValueError(f"level {k} is not in buckets")
            use.append((self._levels.index(k), list(buckets).index(k)))
        use.sort(key=lambda tb: -self._levels[tb[0]])
        n = x.numel()
        dev = x.device
        slots = [self._slots(x, avail, self.tables[t]) for t, _ in use]
        desc = []
        for (t, b), slot in zip(use, slots):
            lv = self.tables[t]
            desc += [slot.data_ptr(), lv.rec.data_ptr(), b]
        desc_t = torch.tensor(desc if desc else [0], dtype=torch.int64, device=dev)
        cell = torch.zeros(n, dtype=torch.int16, device=dev)
        nxt = torch.zeros((n, entries), dtype=torch.int16, device=dev)
        w = torch.zeros((n, entries), dtype=torch.int16, device=dev)
        level = torch.full((n,), -1, dtype=torch.int8, device=dev)
        self.lib("ng_pos_rows", n, i32(len(use)), desc_t, i32(entries), cell, nxt, w, level)
        torch.cuda.current_stream().synchronize()  # desc_t's pointers stay valid until the kernel ran
        return (cell.cpu().numpy(), nxt.cpu().numpy().view(np.uint16), w.cpu().numpy().view(np.uint16),
                level.cpu().numpy())

    def sizes(self) -> list[tuple[int, int, int, int]]:
        """Per level (as built): (k, contexts, pairs, bytes held on the GPU)."""
        out = []
        for lv in self.tables:
            held = (lv.ck, lv.slab, lv.rec, lv.esc[0], lv.esc[1]) + ((lv.thr,) if lv.thr is not None else ())
            b = sum(t.numel() * t.element_size() for t in held)
            out.append((lv.k, lv.contexts, lv.pairs, b))
        return out

    def release(self) -> None:
        """Off the clock: free the tables and the corpus copy."""
        self.released = True
        self.tables = []
        self.tok = None
