"""Exact n-gram counts of the query contexts over a training corpus on one MI355X: the mirror of the record's GPU
counts build, record_367_gpu_counts/track_1_short/counts/build.py (`CountBuild` :161-403, `QueryIndex` :99-141,
`queries` :144-158), on the record flavour of our C ABI (libngram_amd_record.so: 25-bit context ids, 41-bit pair keys).

Per level k the query index (the distinct valid query k-contexts in a canonical linear-probing table, a
representative position each); every shard scanned through its levels as one pass (a level probes only the
positions whose context matched at the previous level: a hit bitmap per level); then per level the table's pairs
compacted, sorted by (context, next token), and per query position tot (uint32 bits), dist (at most 65535) and cnt
(the target's count), plus the record's validation rows from ROW_LEVELS (cells, and the 8 most frequent next tokens with
their 15-bit weights). Beyond the record: `levels`, `level_shards` and `topk` are parameters (the one-GPU share of
the record at configuration c3 counts k = 2..8 over every shard and returns each level's top 4 next
tokens per position), and a level whose pair table overflows reruns with twice the slots (the record raises).

One GPU: `world` must be 1 (the owner exchange is then the identity, as the reference's world == 1 path); the
all-to-all and all-reduce of a multi-GPU build are not part of this build."""

from __future__ import annotations

import time

import numpy as np
import torch

from .build import RECORD_LIB_NAME, lib_path
from .data import BOS, HEADER_BYTES, shard_tokens
from .gpu_val_stats import PAIRS as GVS_PAIRS
from .gpu_val_stats import ValIndex, layout
from .lib import Lib, i32, u64
from . import partcount
from .partcount import count_events, emit_region, record_tops, summarize
from .qindex import QueryIndex

GAP = 32
SCAN_BLOCKS_PER_CU = 8  # level-scan blocks (grid-stride) per compute unit (c3 sweep: 8 fastest of 4-32)
LIST_DENSITY = 0.05  # part mode: a level behind a sparser one probes the previous hits as a position list (c3 sweep)
LEVELS = (2, 3, 4, 5, 6, 10, 20)
LEVEL_SHARDS = {2: 103, 3: 370, 4: 370, 5: 370}
PAIRS = {2: (82.17e6, 0.620), 3: (62.30e6, 0.667), 4: (26.39e6, 0.694), 5: (8.99e6, 0.706), 6: (3.17e6, 0.705),
         10: (0.223e6, 0.604), 20: (0.102e6, 0.581)}
SAFETY = 1.6
LOAD = 0.7
MAX_IDS = (1 << 25) - 4096
ROW_LEVELS = (6, 10, 20)
ROW_K = 8
ROW_COUNTS = (2, 3, 5, 9, 17, 33)
ROW_PURITIES = (0.3, 0.5, 0.7, 0.85, 0.95)
# Partitioned counting: a level whose pair table is larger than PART_MIN_BYTES emits its hits' keys, groups them by
# sub-table (the key hash's top bits) and counts them sub-table by sub-table, each sub-table about SUB_BYTES so that it
# stays in the MALL (256 MB Infinity Cache) while its keys are counted; smaller tables are counted directly.
SUB_BYTES = 64 << 20
PART_MIN_BYTES = 128 << 20
EMIT_CHUNK = 1 << 28  # emitted keys held before a flush (at least one shard's positions)
def record_lib() -> Lib:
    """The record flavour of the library (its scan_level, part_*, rank_scatter and pos_outputs signatures)."""
    return Lib(lib_path(RECORD_LIB_NAME))


def pairs_fit(k: int) -> tuple[float, float]:
    """The reference's fit of distinct (context, next) pairs in n tokens for level k (u, beta): the record's PAIRS,
    gpu_val_stats' for levels it lacks, the deepest fit beyond (levels in between take the shallower neighbour)."""
    if k in PAIRS:
        return PAIRS[k]
    if k in GVS_PAIRS:
        return GVS_PAIRS[k]
    known = sorted(set(PAIRS) | set(GVS_PAIRS))
    below = [j for j in known if j < k]
    j = below[-1] if below else known[0]
    return PAIRS.get(j, GVS_PAIRS.get(j))


def queries(val: np.ndarray, blocks: list[np.ndarray], device, lib: Lib):
    """x, tgt, avail of the validation stream `val` (inputs, then one more token) and then each fit block (likewise),
    each block a segment of its own; a BOS starts a segment (build.py:144-158)."""
    parts = [np.asarray(val, np.uint16), *[np.asarray(b, np.uint16) for b in blocks]]
    x = np.concatenate([p[:-1] for p in parts])
    tgt = np.concatenate([p[1:] for p in parts])
    first = np.zeros(len(x), dtype=bool)
    first[np.cumsum([0, *[len(p) - 1 for p in parts[:-1]]])] = True
    x_t = torch.from_numpy(x.view(np.int16)).to(device)
    idx = torch.arange(len(x), device=device)
    start = (x_t.to(torch.int32) & 0xFFFF) == BOS
    start |= torch.from_numpy(first).to(device)
    seg = torch.empty_like(idx)
    lib.cub("inclusive_max", torch.where(start, idx, torch.zeros_like(idx)), seg, len(x))
    return x_t, torch.from_numpy(tgt.view(np.int16)).to(device), (idx - seg + 1).to(torch.int32)


def device_queries(q: torch.Tensor, lib: Lib):
    """x, tgt, avail of a query stream already on the GPU (int16 tensor: the inputs, then the last target)."""
    x = q[:-1]
    n = x.numel()
    idx = torch.arange(n, device=q.device)
    start = (x.to(torch.int32) & 0xFFFF) == BOS
    start[:1] = True
    seg = torch.empty_like(idx)
    lib.cub("inclusive_max", torch.where(start, idx, torch.zeros_like(idx)), seg, n)
    return x, q[1:], (idx - seg + 1).to(torch.int32)


class CountBuild:
    """The record's count build on one GPU. `shards`: shard file paths (read into pinned host memory, then copied by
    start_load/pace) or uint16 arrays. `levels` ascending; `level_shards`: per level, how many leading shards it
    counts; `topk`: per level the first topk ranked next tokens/counts of each position's context (self.top_tok /
    self.top_cnt [len(levels), N, topk]) when > 0. Construct with `from_device` for tokens already in GPU memory.

    `mode` (attribute): "part" (default) counts without global atomics: each level's hits emitted, hash-partitioned
    by a radix sort and counted partition by partition in LDS, then the engine's owner side; "engine" counts in split
    pair tables (keys and u32 counts apart) with global atomics and ranks by per-context selection after one sort
    (libngram_amd.so's ng_* entry points); "record" runs the record's own C ABI
    calls, as its host does (one packed table per level, two sorts); "partitioned" is "record" with the large tables'
    hits emitted, grouped by sub-table and counted sub-table by sub-table."""

    def __init__(self, shards: list, rank: int = 0, world: int = 1, levels=LEVELS, level_shards=None, topk: int = 0,
                 lib: Lib | None = None):
        if world != 1 or rank != 0:
            raise ValueError("this build runs on one GPU: world must be 1 (the owner exchange is out of scope)")
        self.rank, self.world = rank, world
        self.min_cap = 1 << 20
        self.mode = "part"
        self.density: dict[int, float] = {}  # each level's hit density, from the last build with stats
        self._plist = None  # part mode: a shard's listed positions (list scans)
        self.events_of: dict[int, int] = {}  # part mode: each level's events in the last build
        self.contexts_of: dict[int, int] = {}  # part mode: each level's query contexts in the last build
        self.dratio: dict[int, float] = {}  # "part" mode: each level's distinct pairs per event, from the last build
        self.levels = tuple(levels)
        if not self.levels or list(self.levels) != sorted(set(self.levels)) or self.levels[0] < 1:
            raise ValueError(f"levels must ascend from >= 1: {self.levels}")
        ls = LEVEL_SHARDS if level_shards is None else level_shards
        self.topk = topk
        self.lib = lib or record_lib()
        self.elib = Lib()
        self.timing: dict[str, float] = {}
        self.info: dict = {}
        self.events: list = []
        self.host: list = []
        arrays = []
        for s in shards:
            if isinstance(s, (str, bytes)) or hasattr(s, "__fspath__"):
                n = shard_tokens(s)
                a = torch.empty(n, dtype=torch.int16, pin_memory=True)
                a.numpy()[:] = np.fromfile(s, dtype="<i2", count=n, offset=HEADER_BYTES)
                arrays.append(a)
            else:
                arrays.append(torch.from_numpy(np.ascontiguousarray(s, dtype=np.uint16).view(np.int16)))
        self.sizes = [int(a.numel()) for a in arrays]
        self.level_shards = {k: min(len(arrays), ls.get(k, len(arrays))) for k in self.levels}
        self.starts, self.L = layout(self.sizes)
        self.tok = torch.full((self.L,), -1, dtype=torch.int16, device="cuda")
        self.host = arrays
        self.stream = torch.cuda.Stream()  # the copies' stream (default priority)
        self.pending: list = []

    @classmethod
    def from_device(cls, tok: torch.Tensor, sizes: list[int], starts: list[int], levels=LEVELS, level_shards=None,
                    topk: int = 0, lib: Lib | None = None) -> "CountBuild":
        """A build over shards already laid out in GPU memory (`tok` int16 [L] with SENT gaps, layout()'s starts)."""
        self = cls.__new__(cls)
        self.rank, self.world = 0, 1
        self.min_cap = 1 << 20
        self.mode = "part"
        self.density: dict[int, float] = {}  # each level's hit density, from the last build with stats
        self._plist = None  # part mode: a shard's listed positions (list scans)
        self.events_of: dict[int, int] = {}  # part mode: each level's events in the last build
        self.contexts_of: dict[int, int] = {}  # part mode: each level's query contexts in the last build
        self.dratio: dict[int, float] = {}  # "part" mode: each level's distinct pairs per event, from the last build
        self.levels = tuple(levels)
        ls = LEVEL_SHARDS if level_shards is None else level_shards
        self.topk = topk
        self.lib = lib or record_lib()
        self.elib = Lib()
        self.timing, self.info, self.events, self.host, self.pending = {}, {}, [], [], []
        self.sizes, self.starts, self.L = list(sizes), list(starts), int(tok.numel())
        self.level_shards = {k: min(len(sizes), ls.get(k, len(sizes))) for k in self.levels}
        self.tok = tok
        self.stream = torch.cuda.current_stream()
        ev = torch.cuda.Event()
        ev.record()
        self.events = [ev] * len(sizes)
        return self

    def caps(self) -> dict[int, int]:
        """Each level's pair table slots: the estimated pairs of the level's tokens, at LOAD (build.py:205-212)."""
        caps = {}
        for k in self.levels:
            n_k = sum(self.sizes[: self.level_shards[k]])
            u, beta = pairs_fit(k)
            caps[k] = max(self.min_cap, int(min(SAFETY * u * (max(n_k, 1) / 4e8) ** beta, n_k) / LOAD))
        return caps

    def prepare(self) -> None:
        """Before the clock: the caching allocator's blocks for the pair tables (no collectives on one GPU)."""
        warm = torch.empty(int(1.33 * sum(9 * cap for cap in self.caps().values())), dtype=torch.uint8, device="cuda")
        del warm
        torch.cuda.synchronize()

    def start_load(self, steps: int = 1) -> None:
        """The host shards' copies split into `steps` equal shares, the first enqueued (build.py:231-243)."""
        self.pending = []
        for a, st in zip(self.host, self.starts):
            n = a.numel()
            for lo in range(0, max(n, 1), 4 << 20):  # an empty shard: one empty copy, so that it has its event too
                hi = min(n, lo + (4 << 20))
                self.pending.append((st + lo, a, lo, hi, hi == n))
        self.pending.reverse()
        self.per_step = -(-len(self.pending) // max(1, steps))
        self.events = []
        self.load_start = torch.cuda.Event(enable_timing=True)
        self.load_start.record(self.stream)
        self.pace()

    def pace(self) -> None:
        """The next share of the copies (build.py:245-255)."""
        with torch.cuda.stream(self.stream):
            for _ in range(min(self.per_step, len(self.pending))):
                at, a, lo, hi, last = self.pending.pop()
                self.tok[at : at + hi - lo].copy_(a[lo:hi], non_blocking=True)
                if last:
                    ev = torch.cuda.Event(enable_timing=True)
                    ev.record(self.stream)
                    self.events.append(ev)

    def load_ms(self) -> float:
        """The copies' time on the device from start_load to the last shard's copy, once all are enqueued
        (build.py:257-259)."""
        if self.pending or not self.events or getattr(self, "load_start", None) is None:
            raise ValueError("the loads have not all been enqueued")
        self.events[-1].synchronize()
        return self.load_start.elapsed_time(self.events[-1])

    def _event(self, name: str, k: int, i: int, n: int):
        """A pair of timing events around a launch (recorded on the current stream), kept in kernel_events."""
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        self.kernel_events.append((name, k, i, n, e0, e1))
        return e0, e1

    def _scan(self, index, tables, bms, shard_ids, levels) -> None:
        lib, grid = self.lib, self.grid
        for i in shard_ids:
            st, n = self.starts[i], self.sizes[i]
            n32 = (n + 31) // 32 * 32
            torch.cuda.current_stream().wait_event(self.events[i])
            scanned = [k for k in self.levels if i < self.level_shards[k]]
            for li, k in enumerate(scanned):
                if k not in levels:
                    continue
                vi = index[k]
                t = tables[k]
                # gated by this shard's previous scanned level; a shard that level skipped is probed whole
                bm_in = None if li == 0 else bms[scanned[li - 1]][st // 32 :]
                if self.mode == "engine":
                    e0, e1 = self._event("scan_count", k, i, n32)
                    e0.record()
                    self.elib("ng_scan_count", self.tok[st:], n32, i32(k), bm_in, bms[k][st // 32 :], vi.table,
                              u64(vi.cap), vi.rep, self.x, t["keys"], t["cnts"], u64(t["cap"]), t["flags"], i32(grid),
                              i32(self._scan_mode(li, scanned)))
                    e1.record()
                elif t["pbits"]:
                    if t["pending"] + n32 > t["emit"].numel():
                        self._flush(t, k)
                    e0, e1 = self._event("scan_emit", k, i, n32)
                    e0.record()
                    lib("scan_emit", self.tok[st:], n32, i32(k), bm_in, bms[k][st // 32 :], vi.table, u64(vi.cap),
                        vi.rep, self.x, t["flags"], i32(grid), i32(0), t["emit"], t["emitted"])
                    e1.record()
                    t["pending"] += n32
                else:
                    e0, e1 = self._event("scan_level", k, i, n32)
                    e0.record()
                    lib("scan_level", self.tok[st:], n32, i32(k), bm_in, bms[k][st // 32 :], vi.table, u64(vi.cap),
                        vi.rep, self.x, t["pk"], t["pc"], u64(t["cap"]), t["flags"], i32(grid),
                        i32(int(li > 0 and k > 5)))
                    e1.record()
        for k in levels:
            if tables[k]["pbits"]:
                self._flush(tables[k], k)

    def _scan_mode(self, li: int, scanned: list, lists: bool = False) -> int:
        """The engine scan's mode for a shard's li-th scanned level: a lane per position (0) for the first level and
        behind a dense previous level, else the LDS-listed set positions (2), or with `lists` (part mode) below
        LIST_DENSITY the set positions listed in memory first (3). The previous level's density is the one its last
        build measured (stats), dense when unknown."""
        if li == 0:
            return 0
        d = self.density.get(scanned[li - 1])
        if d is None or d >= 0.5:
            return 0
        return 3 if lists and d < LIST_DENSITY else 2

    def _flush(self, t: dict, k: int) -> None:
        """Count a partitioned level's emitted keys: group them by sub-table, then count sub-table by sub-table."""
        if t["pending"] == 0:
            return
        lib = self.lib
        n = int(t["emitted"].item())
        if getattr(self, "grouped", None) is None or self.grouped.numel() < t["emit"].numel():
            self.grouped = torch.empty(t["emit"].numel(), dtype=torch.int64, device=t["emit"].device)
        if n:
            pbits = t["pbits"]
            counts = torch.zeros(1 << pbits, dtype=torch.int64, device=t["pk"].device)
            e0, e1 = self._event("group", k, -1, n)
            e0.record()
            lib("subpart_count", t["emit"], n, i32(pbits), counts)
            cursor = torch.cumsum(counts, 0) - counts
            lib("subpart_scatter", t["emit"], n, i32(pbits), cursor, self.grouped)
            e1.record()
            e0, e1 = self._event("aggregate", k, -1, n)
            e0.record()
            lib("aggregate", self.grouped, n, t["pk"], t["pc"], u64(t["sub_cap"]), i32(pbits), t["flags"],
                i32(self.grid))
            e1.record()
        t["emitted"].zero_()
        t["pending"] = 0

    def counts(self, x: torch.Tensor, tgt: torch.Tensor, avail: torch.Tensor, stats: bool = False) -> torch.Tensor:
        """int32 [3, len(levels), len(x)]: per query position and level its context's total occurrences (uint32 bits),
        distinct next tokens (at most 65535) and its target's count; also the rows (batch_rows) and, with topk, the
        per-level top next tokens (build.py:261-388). `stats`: also count each level's corpus hits (self.info)."""
        self.stats = stats
        lib, timing, info = self.lib, self.timing, self.info
        dev = self.tok.device

        def lap(name: str) -> None:
            torch.cuda.current_stream().synchronize()
            now = time.perf_counter()
            timing[name] = timing.get(name, 0.0) + now - lap.t
            lap.t = now

        lap.t = time.perf_counter()
        self.kernel_events = []
        self.x = x
        N = x.numel()
        self.grid = torch.cuda.get_device_properties(dev).multi_processor_count * SCAN_BLOCKS_PER_CU
        if self.mode == "part":
            return self._counts_part(x, avail, tgt, N, lap)
        if self.mode == "engine":
            index = {k: QueryIndex(self.elib, x, avail, k) for k in self.levels}
        else:
            index = {k: ValIndex(lib, x, avail, k, max_ids=MAX_IDS) for k in self.levels}
        lap("index")
        caps = self.caps()
        tables = {}
        chunk = max([EMIT_CHUNK] + [(n + 31) // 32 * 32 for n in self.sizes])
        for k in self.levels:
            tables[k] = self._table(caps[k], dev, chunk)
        nwords = self.L // 32
        bms = {k: torch.zeros(nwords, dtype=torch.int32, device=dev) for k in self.levels}
        self._scan(index, tables, bms, range(len(self.sizes)), set(self.levels))
        reruns = {k: 0 for k in self.levels}
        while True:
            fl = {k: tables[k]["flags"].cpu().tolist() for k in self.levels}
            over = [k for k in self.levels if fl[k][0]]
            if not over:
                break
            for k in over:  # the bitmaps are whole: only the overflowed level reruns, with twice the slots
                reruns[k] += 1
                tables[k] = self._table(2 * tables[k]["cap"], dev, chunk)
            self._scan(index, tables, bms, range(len(self.sizes)), set(over))
        lap("scan")
        hits = {k: int(self._popcount(bms[k]).item()) for k in self.levels} if self.stats else {}
        for k, h in hits.items():
            n_k = sum(self.sizes[: self.level_shards[k]])
            self.density[k] = h / max(1, n_k)
        del bms
        out = torch.zeros((3, len(self.levels), N), dtype=torch.int32, device=dev)
        rows = all(k in self.levels for k in ROW_LEVELS)
        if rows:
            row_entries = torch.zeros((len(ROW_LEVELS), N, ROW_K), dtype=torch.int32, device=dev)
            row_top = torch.zeros((len(ROW_LEVELS), N), dtype=torch.int32, device=dev)
        if self.topk:
            self.top_tok = torch.zeros((len(self.levels), N, self.topk), dtype=torch.int16, device=dev)
            self.top_cnt = torch.zeros((len(self.levels), N, self.topk), dtype=torch.int32, device=dev)
        for li, k in enumerate(self.levels):
            vi = index.pop(k)
            t = tables.pop(k)
            want = max(self.topk, ROW_K if (rows and k in ROW_LEVELS) else 0)
            if self.mode == "engine":
                U, tot, top_tok, top_cnt, want = self._outputs_engine(li, k, vi, t, tgt, out, want)
            else:
                U, tot, top_tok, top_cnt = self._outputs_record(li, k, vi, t, tgt, out, want)
            self._level_rows(k, vi, want, tot, top_tok, top_cnt, row_entries if rows else None,
                             row_top if rows else None)
            del top_tok, top_cnt
            info[k] = dict(contexts=vi.n, ids=vi.ids, pairs=U, cap=t["cap"], pbits=t["pbits"], hits=hits.get(k),
                           reruns=reruns[k])
            del t, tot, vi
        lap("outputs")
        if rows:
            self._rows(out, row_entries, row_top, N)
            lap("rows")
        self.out = out
        return out

    def _level_rows(self, k, vi, want, tot, top_tok, top_cnt, row_entries, row_top) -> None:
        """A level's share of the rows (its top ROW_K entries per position, if k is a row level) and the uint32 check
        of its totals."""
        if row_entries is not None and k in ROW_LEVELS:
            ri = ROW_LEVELS.index(k)
            ctx = vi.ctx_of.long()
            at = ((ctx >= 0) & (ctx < vi.ids)).nonzero().squeeze(1)
            c = ctx[at]
            tt = top_tok.view(-1, want)[c, :ROW_K].to(torch.int32) & 0xFFFF
            tc = top_cnt.view(-1, want)[c, :ROW_K].to(torch.int64)
            top = tc[:, :1].clamp_min(1)
            # the weights as the model reads them (15 bits): scaled down where the top count is larger
            w = torch.where(top > 32767, (tc * 32767 + top - 1) // top, tc)
            row_entries[ri, at] = torch.where(tc > 0, tt | (w.to(torch.int32) << 16), 0)
            row_top[ri, at] = tc[:, 0].clamp_max((1 << 31) - 1).to(torch.int32)
        if tot is not None and vi.ids and int(tot.max().item()) >= 1 << 32:
            raise RuntimeError(f"k={k}: a total does not fit uint32")

    def _counts_part(self, x, avail, tgt, N, lap) -> torch.Tensor:
        """counts() in "part" mode: level after level, every shard's scan emits its hits (no global atomics), the
        hits are hash-partitioned by a radix sort of their mixed keys and counted partition by partition in LDS
        (the query positions' target counts answered there too); then the owner side of the engine mode. A level's
        query index holds only the positions whose previous level's context occurred (when the level counts no
        shard the previous one skips): a context occurs only where its suffix does, so the others stay zero."""
        dev, info = self.tok.device, self.info
        nwords = self.L // 32
        bms = {k: torch.zeros(nwords, dtype=torch.int32, device=dev) for k in self.levels}
        out = torch.zeros((3, len(self.levels), N), dtype=torch.int32, device=dev)
        rows = all(k in self.levels for k in ROW_LEVELS)
        row_entries = row_top = None
        if rows:
            row_entries = torch.zeros((len(ROW_LEVELS), N, ROW_K), dtype=torch.int32, device=dev)
            row_top = torch.zeros((len(ROW_LEVELS), N), dtype=torch.int32, device=dev)
        if self.topk:
            self.top_tok = torch.zeros((len(self.levels), N, self.topk), dtype=torch.int16, device=dev)
            self.top_cnt = torch.zeros((len(self.levels), N, self.topk), dtype=torch.int32, device=dev)
        G = self.grid
        R = max(emit_region((n + 31) // 32 * 32, G) for n in self.sizes)
        span = self.starts[-1] + (self.sizes[-1] + 31) // 32 * 32 - self.starts[0] if self.sizes else 0
        # room for one region per shard and block, or for one scan over every shard (a list scan's regions included)
        n_reg = max(len(self.sizes) * G * R, G * emit_region(span, G), G * (-(-max(span, 1) // (G * 256)) * 256))
        regions = torch.empty(n_reg, dtype=torch.int64, device=dev)
        scan_t = count_t = index_t = 0.0
        for li, k in enumerate(self.levels):
            t0 = time.perf_counter()
            prev = self.levels[li - 1] if li else None
            seen = None
            if prev is not None and self.level_shards[k] <= self.level_shards[prev]:
                seen = torch.nonzero(out[1, li - 1] > 0).squeeze(1).to(torch.int32)
            vi = QueryIndex(self.elib, x, avail, k, seen, expect=self.contexts_of.get(k))
            self.contexts_of[k] = vi.n
            index_t += time.perf_counter() - t0
            t0 = time.perf_counter()
            seg = self._part_emit(k, vi, bms, regions, R)
            t1 = time.perf_counter()
            ev_fn = lambda name, n, k=k: self._event(name, k, -1, n)  # noqa: E731
            c = count_events(self.elib, self.lib, None, 0, vi.ids, self.dratio.get(k, 1.0), (vi.ctx_of, tgt, seen),
                             event=ev_fn, seg=seg, presort="ctx")
            del seg
            n_ev = c.n_ev
            self.events_of[k] = n_ev
            self.dratio[k] = c.U / max(1, n_ev)
            t2 = time.perf_counter()
            scan_t += t1 - t0
            count_t += t2 - t1
            want = max(self.topk, ROW_K if (rows and k in ROW_LEVELS) else 0)
            if c.cb:
                tot, top_tok, top_cnt, want = self._owner_packed(li, k, vi, c, tgt, out, want,
                                                                 rows and k in ROW_LEVELS)
            else:  # pairs unpacked (more large counts than the escape table held)
                tot, top_tok, top_cnt, want = self._owner(li, k, vi, c.pairs, c.counts, c.U, tgt, out, want,
                                                          qcnt=c.qcnt)
            self._level_rows(k, vi, want, tot, top_tok, top_cnt, row_entries, row_top)
            info[k] = dict(contexts=vi.n, ids=vi.ids, pairs=c.U, events=n_ev, pbits=c.pbits, cap=0, hits=None,
                           reruns=0)
            del tot, top_tok, top_cnt, vi, c, seen
        del regions
        if self.stats:
            for k in self.levels:
                h = int(self._popcount(bms[k]).item())
                info[k]["hits"] = h
                self.density[k] = h / max(1, sum(self.sizes[: self.level_shards[k]]))
        del bms
        lap("outputs")
        self.timing["part_index_host"] = self.timing.get("part_index_host", 0.0) + index_t
        self.timing["part_scan_host"] = self.timing.get("part_scan_host", 0.0) + scan_t
        self.timing["part_count_host"] = self.timing.get("part_count_host", 0.0) + count_t
        if rows:
            self._rows(out, row_entries, row_top, N)
            lap("rows")
        self.out = out
        return out

    def _part_emit(self, k, vi, bms, regions, R):
        """Level k's scan of every shard it counts, hits emitted to per-block regions with each block's top-digit
        histogram: count_events' seg = (regions, R, ev_count, dhist, nseg, flags)."""
        elib, dev, G = self.elib, self.tok.device, self.grid
        shards = [i for i in range(len(self.sizes)) if i < self.level_shards[k]]
        nseg = len(shards) * G
        ev_count = torch.zeros(max(nseg, 1), dtype=torch.int32, device=dev)
        # the scan's digit histograms only where the last build's events let the partition sort read the regions
        last = self.events_of.get(k)
        dhist = torch.empty(256 * max(nseg, 1), dtype=torch.int32, device=dev) \
            if last is None or last >= partcount.SEG_MIN_EVENTS * nseg else None
        flags = torch.zeros(2, dtype=torch.int32, device=dev)
        scans = {tuple(q for q in self.levels if i < self.level_shards[q]) for i in shards}
        if len(shards) > 1 and len(scans) == 1:
            # every shard scans the same levels: one launch over all of them (the SENT gaps between shards hold no
            # context), except for a first level whose shards may still be arriving from the host (each shard's scan
            # then starts once its own copy is done)
            scanned = list(scans.pop())
            si = scanned.index(k)
            if si > 0 or not self.host:
                return self._part_emit_all(k, vi, None if si == 0 else bms[scanned[si - 1]], bms[k], shards, regions,
                                           flags, self._scan_mode(si, scanned, lists=True))
        for j, i in enumerate(shards):
            st, n = self.starts[i], self.sizes[i]
            n32 = (n + 31) // 32 * 32
            torch.cuda.current_stream().wait_event(self.events[i])
            scanned = [q for q in self.levels if i < self.level_shards[q]]
            si = scanned.index(k)
            # gated by this shard's previous scanned level; a shard that level skipped is probed whole
            bm_in = None if si == 0 else bms[scanned[si - 1]][st // 32 :]
            mode = self._scan_mode(si, scanned, lists=True)
            if mode == 3:  # the previous level's hits listed, then probed one lane each
                if self._plist is None or self._plist.numel() < n32:
                    self._plist = torch.empty(max(self.sizes) + 64, dtype=torch.int64, device=dev)
                n_list = torch.zeros(1, dtype=torch.int64, device=dev)
                b0, b1 = self._event("bits_list", k, i, n32)
                b0.record()
                elib.cub("ng_bits_list", bm_in, n32 // 32, self._plist, n_list)
                b1.record()
            e0, e1 = self._event("scan_emit", k, i, n32)
            e0.record()
            if mode == 3:
                elib("ng_scan_emit_list", self.tok[st:], self._plist, n_list, i32(k), vi.table, u64(vi.cap), vi.rep,
                     self.x, bms[k][st // 32 :], regions[j * G * R :], u64(R), ev_count[j * G :], flags, i32(G),
                     dhist[j * G :] if dhist is not None else None, nseg)
            else:
                elib("ng_scan_emit", self.tok[st:], n32, i32(k), bm_in, bms[k][st // 32 :], vi.table, u64(vi.cap),
                     vi.rep, self.x, regions[j * G * R :], u64(R), ev_count[j * G :], flags, i32(G), i32(mode),
                     dhist[j * G :] if dhist is not None else None, nseg)
            e1.record()
        return regions, R, ev_count, dhist, nseg, flags  # count_events checks the flags with its first read

    def _part_emit_all(self, k, vi, bm_in, bm_out, shards, regions, flags, mode):
        """_part_emit of a level whose shards all scan the same levels, in one launch over all of them (from the first
        shard's start to the last one's end): a lane per position (mode 0), the LDS-listed set positions (2), or one
        position list of the previous level's set bits and one list scan (3), instead of one of each per shard;
        seg = (regions, R, ev_count, dhist, grid, flags)."""
        elib, dev, G = self.elib, self.tok.device, self.grid
        lo = self.starts[shards[0]]
        hi = self.starts[shards[-1]] + (self.sizes[shards[-1]] + 31) // 32 * 32
        for i in shards:
            torch.cuda.current_stream().wait_event(self.events[i])
        n = hi - lo
        if mode == 3:
            R = -(-max(n, 1) // (G * 256)) * 256  # a list scan's block emits at most 256 per round
        else:
            R = emit_region(n, G)
        if G * R > regions.numel():
            raise RuntimeError(f"k={k}: the emit regions are too small for one scan over every shard")
        ev_count = torch.zeros(G, dtype=torch.int32, device=dev)
        last = self.events_of.get(k)
        dhist = torch.empty(256 * G, dtype=torch.int32, device=dev) \
            if last is None or last >= partcount.SEG_MIN_EVENTS * G else None
        if mode == 3:
            if self._plist is None or self._plist.numel() < n:
                self._plist = torch.empty(n + 64, dtype=torch.int64, device=dev)
            n_list = torch.zeros(1, dtype=torch.int64, device=dev)
            b0, b1 = self._event("bits_list", k, -1, n)
            b0.record()
            elib.cub("ng_bits_list", bm_in[lo // 32 :], n // 32, self._plist, n_list)
            b1.record()
        e0, e1 = self._event("scan_emit", k, -1, n)
        e0.record()
        if mode == 3:
            elib("ng_scan_emit_list", self.tok[lo:], self._plist, n_list, i32(k), vi.table, u64(vi.cap), vi.rep,
                 self.x, bm_out[lo // 32 :], regions, u64(R), ev_count, flags, i32(G), dhist, G)
        else:
            elib("ng_scan_emit", self.tok[lo:], n, i32(k), None if bm_in is None else bm_in[lo // 32 :],
                 bm_out[lo // 32 :], vi.table, u64(vi.cap), vi.rep, self.x, regions, u64(R), ev_count, flags, i32(G),
                 i32(mode), dhist, G)
        e1.record()
        return regions, R, ev_count, dhist, G, flags

    def _owner_packed(self, li, k, vi, c, tgt, out, want, zero_tops):
        """The owner side from packed pairs: per present context its record (sorted by context, keys only), then per
        query position its context's record and counted target (ng_pos_summary)."""
        N, n_own = vi.ctx_of.numel(), vi.ids
        ktop = 1 if want <= 1 else 2 if want <= 2 else 4 if want <= 4 else 8
        try:
            sm = summarize(self.elib, self.lib, c, n_own, ktop, zero_tops, lambda name, n: self._event(name, k, -1, n))
            rec, dist = sm.rec, sm.dist
        except RuntimeError as e:
            raise RuntimeError(f"k={k}: {e}") from None
        e0, e1 = self._event("pos_gather", k, -1, N)
        e0.record()
        kout = self.topk
        self.elib("ng_pos_summary", vi.ctx_of, N, 0, n_own, tgt, rec, dist, None, c.qcnt, i32(ktop), i32(kout),
                  i32(li), out[0, li], out[1, li], out[2, li], self.top_tok[li] if kout else None,
                  self.top_cnt[li] if kout else None, None)
        e1.record()
        top_tok = top_cnt = None
        if zero_tops:
            top_tok, top_cnt = record_tops(rec, ktop)
        return None, top_tok, top_cnt, ktop

    def _outputs_engine(self, li, k, vi, t, tgt, out, want):
        """One level's outputs with the engine: the split table compacted, its pairs sorted by context, per-context
        totals and top entries by selection, then one gather per query position (the target's count looked up in the
        split table)."""
        elib, lib, dev = self.elib, self.lib, self.tok.device
        N, lo, hi = vi.ctx_of.numel(), 0, vi.ids
        counter = torch.zeros(1, dtype=torch.int64, device=dev)
        cap = t["cap"]
        U_max = cap
        ck = torch.empty(U_max, dtype=torch.int64, device=dev)
        cc = torch.empty(U_max, dtype=torch.int32, device=dev)
        e0, e1 = self._event("compact", k, -1, cap)
        e0.record()
        elib("ng_table_compact", t["keys"], t["cnts"], u64(cap), ck, cc, counter)
        e1.record()
        U = int(counter.item())
        tot, top_tok, top_cnt, want = self._owner(li, k, vi, ck, cc, U, tgt, out, want, t=t)
        t.pop("keys"), t.pop("cnts")
        return U, tot, top_tok, top_cnt, want

    def _owner(self, li, k, vi, ck, cc, U, tgt, out, want, t=None, qcnt=None):
        """A level's owner side from its U distinct pairs (ck, cc; consumed): sorted by context, per-context totals
        and top entries by selection, then one gather per query position (the target's count from qcnt, or looked
        up in the split table t)."""
        elib, lib, dev = self.elib, self.lib, self.tok.device
        N, lo, hi = vi.ctx_of.numel(), 0, vi.ids
        n_own = hi - lo
        ctx_bits = max(1, (max(n_own, 2) - 1).bit_length())
        uk, agg = torch.empty(U, dtype=torch.int64, device=dev), torch.empty(U, dtype=torch.int32, device=dev)
        e0, e1 = self._event("sort", k, -1, U)
        e0.record()
        if U:  # by context only: the target's count is looked up apart, the ranking needs no token order
            lib.cub("sort_pairs", ck, uk, cc, agg, U, i32(16), i32(16 + ctx_bits))
        e1.record()
        del ck, cc
        start = torch.zeros(n_own, dtype=torch.int64, device=dev)
        end = torch.zeros(n_own, dtype=torch.int64, device=dev)
        ktop = 1 if want <= 1 else 2 if want <= 2 else 4 if want <= 4 else 8
        tot = torch.empty(n_own, dtype=torch.int64, device=dev)
        top_tok = torch.zeros(n_own * ktop, dtype=torch.int16, device=dev)
        top_cnt = torch.zeros(n_own * ktop, dtype=torch.int32, device=dev)
        e0, e1 = self._event("ctx_topk", k, -1, U)
        e0.record()
        lib("seg_bounds", uk, U, start, end)
        elib("ng_ctx_topk", uk, agg, start, end, n_own, i32(ktop), tot, top_tok, top_cnt)
        e1.record()
        e0, e1 = self._event("pos_gather", k, -1, N)
        e0.record()
        kout = self.topk
        pk, pc, cap = (t["keys"], t["cnts"], t["cap"]) if qcnt is None else (None, None, 0)
        elib("ng_pos_gather", vi.ctx_of, N, lo, hi, tgt, uk, agg, start, end, tot, top_tok, top_cnt, None, pk, pc,
             u64(cap), qcnt, i32(ktop), i32(kout), i32(li), out[0, li], out[1, li], out[2, li],
             self.top_tok[li] if kout else None, self.top_cnt[li] if kout else None, None)
        e1.record()
        return tot, top_tok, top_cnt, ktop

    def _outputs_record(self, li, k, vi, t, tgt, out, want):
        """One level's outputs with the record's calls: part_count/part_scatter, sort by pair key, seg_bounds,
        ctx_tot, pos_outputs, and for top entries rank_keys + a stable sort + rank_scatter (build.py:307-371)."""
        lib, dev = self.lib, self.tok.device
        N, lo, hi = vi.ctx_of.numel(), 0, vi.ids
        pk, pc, cap = t.pop("pk"), t.pop("pc"), t["cap"]
        bounds = torch.tensor([lo, hi], dtype=torch.int64, device=dev)
        cnt = torch.zeros(1, dtype=torch.int64, device=dev)
        lib("part_count", pk, u64(cap), bounds, i32(1), cnt)
        U = int(cnt.item())
        cursor = torch.zeros(1, dtype=torch.int64, device=dev)
        send_k = torch.empty(U, dtype=torch.int64, device=dev)
        send_c = torch.empty(U, dtype=torch.int32, device=dev)
        lib("part_scatter", pk, pc, u64(cap), bounds, i32(1), cursor, send_k, send_c)
        del pk, pc
        n_own = hi - lo
        ctx_bits = max(1, (max(n_own, 2) - 1).bit_length())
        uk, agg = torch.empty_like(send_k), torch.empty_like(send_c)
        if U:  # one GPU: the table's keys are already distinct (no reduce_by_key)
            lib.cub("sort_pairs", send_k, uk, send_c, agg, U, i32(0), i32(16 + ctx_bits))
        del send_k, send_c
        start = torch.zeros(n_own, dtype=torch.int64, device=dev)
        end = torch.zeros(n_own, dtype=torch.int64, device=dev)
        lib("seg_bounds", uk, U, start, end)
        tot = torch.empty(n_own, dtype=torch.int64, device=dev)
        lib("ctx_tot", start, end, agg, n_own, tot)
        lib("pos_outputs", vi.ctx_of, N, lo, hi, tgt, uk, agg, start, end, tot, out[0, li], out[1, li], out[2, li])
        top_tok = top_cnt = None
        if want:
            key2 = torch.empty(U, dtype=torch.int64, device=dev)
            val2 = torch.empty(U, dtype=torch.int32, device=dev)
            lib("rank_keys", uk, agg, U, key2, val2)
            k2s, sv = torch.empty_like(key2), torch.empty_like(val2)
            if U:
                lib.cub("sort_pairs", key2, k2s, val2, sv, U, i32(0), i32(32 + ctx_bits))
            del key2, val2, k2s
            top_tok = torch.zeros(n_own * want, dtype=torch.int16, device=dev)
            top_cnt = torch.zeros(n_own * want, dtype=torch.int32, device=dev)
            lib("rank_scatter", sv, U, uk, agg, start, top_tok, top_cnt, i32(want))
            del sv
            if self.topk:
                lib("pos_topk", vi.ctx_of, N, lo, hi, top_tok, top_cnt, i32(want), i32(self.topk), self.top_tok[li],
                    self.top_cnt[li])
        return U, tot, top_tok, top_cnt

    def _table(self, cap: int, dev, chunk: int) -> dict:
        """A level's pair table of at least `cap` slots: split (engine), packed and counted directly (record), or
        (partitioned, larger than PART_MIN_BYTES) packed in 2^pbits sub-tables of about SUB_BYTES with an emit buffer
        of `chunk` keys."""
        if self.mode == "engine":
            return {"keys": torch.full((cap,), -1, dtype=torch.int64, device=dev),
                    "cnts": torch.zeros(cap, dtype=torch.int32, device=dev), "cap": cap, "pbits": 0,
                    "flags": torch.zeros(2, dtype=torch.int32, device=dev), "pending": 0}
        pbits, sub_cap = 0, cap
        if self.mode == "partitioned" and cap * 8 > PART_MIN_BYTES:
            pbits = min(int(self.lib.plain("max_pbits")), max(1, -(-(cap * 8) // SUB_BYTES) - 1).bit_length())
            sub_cap = -(-cap // (1 << pbits))
            cap = sub_cap << pbits
        t = {"pk": torch.full((cap,), -1, dtype=torch.int64, device=dev),
             "pc": torch.zeros((cap + 3) // 4, dtype=torch.int32, device=dev), "cap": cap, "pbits": pbits,
             "sub_cap": sub_cap, "flags": torch.zeros(2, dtype=torch.int32, device=dev), "pending": 0}
        if pbits:
            t["emit"] = torch.empty(chunk, dtype=torch.int64, device=dev)
            t["emitted"] = torch.zeros(1, dtype=torch.int64, device=dev)
        return t

    def _popcount(self, bm: torch.Tensor) -> torch.Tensor:
        # bit count of an int32 bitmap, in torch (a byte table lookup)
        table = torch.tensor([bin(i).count("1") for i in range(256)], dtype=torch.int64, device=bm.device)
        b = bm.view(torch.uint8).long()
        return table[b].sum()

    def _rows(self, out, row_entries, row_top, N) -> None:
        """Per position its cell (0: no match at ROW_LEVELS[0]) and the ROW_K candidates of its deepest matched level
        (build.py:376-387)."""
        dev = out.device
        tot = out[0, [self.levels.index(k) for k in ROW_LEVELS]].to(torch.int64) & 0xFFFFFFFF
        depth = ((tot > 0).to(torch.int64) * torch.arange(1, len(ROW_LEVELS) + 1, device=dev)[:, None]).amax(0) - 1
        sel = depth.clamp_min(0)
        pos = torch.arange(N, device=dev)
        total = tot[sel, pos].double()
        share = row_top[sel, pos].double() / total.clamp_min(1)
        count_bin = sum((total >= e).to(torch.int64) for e in ROW_COUNTS)
        purity = sum((share >= e).to(torch.int64) for e in ROW_PURITIES)
        cell = (((1 + depth) * (len(ROW_COUNTS) + 1) + count_bin) * (len(ROW_PURITIES) + 1) + purity) * (depth >= 0)
        self.row_cells = cell.to(torch.int32)
        self.row_entries = torch.where((depth >= 0)[:, None], row_entries[sel, pos], 0)

    def batch_rows(self, at: int, n: int, capacity: int) -> torch.Tensor:
        """The record's rows of the n query positions from `at`: their cells, then `capacity` entries (position,
        token | count << 16), padded with (i % n, 0) (build.py:390-403)."""
        cell, e = self.row_cells[at : at + n], self.row_entries[at : at + n]
        pos, k = (e != 0).nonzero(as_tuple=True)
        m = pos.numel()
        if m > capacity:
            raise AssertionError(f"{m} candidates overflow the rows' {capacity} entries")
        rows = torch.zeros(n + 2 * capacity, dtype=torch.int32, device=e.device)
        rows[:n] = cell
        ent = rows[n:].view(-1, 2)
        ent[:, 0] = torch.arange(capacity, device=e.device, dtype=torch.int32) % n
        ent[:m, 0] = pos.to(torch.int32)
        ent[:m, 1] = e[pos, k]
        return rows
