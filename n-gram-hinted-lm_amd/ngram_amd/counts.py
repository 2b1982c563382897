"""The record's GPU count build on one MI355X: `CountBuild` with the surface of
record_367_gpu_counts/track_1_short/counts/build.py (CountBuild :161-403, queries :144-158) on the engine's level
pipeline (levels.LevelBuild).

  * construct: the shards read into pinned host memory (or taken from arrays), their device buffer laid out by
    data.pack_layout (SENT gaps), nothing copied yet;
  * start_load(steps) / pace(): the host-to-device copies split into `steps` equal shares, one share enqueued per call
    on a copy stream of default priority; each shard's first scan waits for that shard's last copy only;
  * counts(x, tgt, avail) -> int32 [3, len(levels), N]: per query position and level its context's total
    occurrences (uint32 bits), distinct next tokens (at most 65535) and the target's count (no TOP rule, as the
    record's pos_outputs :411-429); with `topk`, each level's first topk next tokens and counts (self.top_tok,
    self.top_cnt [len(levels), N, topk]); when every ROW_LEVELS level is counted, the record's rows (row_cells int32
    [N], row_entries int32 [N, ROW_K]) made on the GPU by ng_record_rows;
  * batch_rows(at, n, capacity): a training batch's rows, ng_batch_rows.

Beyond the record: `levels`, `level_shards` and `topk` are parameters (BASELINE configuration c3 counts k = 2..8 over
every shard with top-4), and `from_device` builds over tokens already in GPU memory. One GPU: `world` must be 1."""

from __future__ import annotations

import numpy as np
import torch

from . import data
from .lib import Lib, i32
from .levels import LevelBuild

LEVELS = (2, 3, 4, 5, 6, 10, 20)
LEVEL_SHARDS = {2: 103, 3: 370, 4: 370, 5: 370}  # the record's shard caps of the short levels (build.py:52-53)
ROW_LEVELS = (6, 10, 20)
ROW_K = 8
COPY_TOKENS = 4 << 20  # tokens per host-to-device copy


def queries(val: np.ndarray, blocks: list, device, lib: Lib | None = None):
    """x, tgt, avail of the validation stream `val` (its inputs, then one more token) followed by each fit block
    (likewise): one segment per part, and a new segment at every BOS. `lib` is accepted for the reference's signature;
    the segments are computed on the host (data.segments)."""
    parts = [np.asarray(p, np.uint16) for p in (val, *blocks)]
    x = np.concatenate([p[:-1] for p in parts])
    tgt = np.concatenate([p[1:] for p in parts])
    breaks = np.cumsum([len(p) - 1 for p in parts[:-1]]).tolist()
    avail = data.segments(x, breaks)
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    return to(x.view(np.int16)), to(tgt.view(np.int16)), to(avail)


def device_queries(q: torch.Tensor, lib: Lib | None = None):
    """x, tgt, avail of one query stream already on the GPU (int16: the inputs, then the last target)."""
    x = q[:-1]
    avail = data.segments(x.cpu().numpy().view(np.uint16))
    return x, q[1:], torch.from_numpy(avail).to(q.device)


def _pinned(s) -> torch.Tensor:
    """A shard (file path or uint16 array) as an int16 tensor in pinned host memory."""
    a = data.read_shard(s) if isinstance(s, (str, bytes)) or hasattr(s, "__fspath__") else np.asarray(s, np.uint16)
    t = torch.empty(len(a), dtype=torch.int16, pin_memory=True)
    if len(a):
        t.numpy()[:] = np.asarray(a).view(np.int16)
    return t


class CountBuild:
    """The record's count build on one GPU (see the module docstring). `shards`: shard file paths or uint16 arrays."""

    def __init__(self, shards: list, rank: int = 0, world: int = 1, levels=LEVELS, level_shards=None, topk: int = 0,
                 lib: Lib | None = None):
        if world != 1 or rank != 0:
            raise ValueError("this build runs on one GPU: world must be 1 (the owner exchange is out of scope)")
        self.rank, self.world = rank, world
        self.host = [_pinned(s) for s in shards]
        sizes = [int(h.numel()) for h in self.host]
        starts, L = data.pack_layout(sizes)
        tok = torch.full((L,), -1, dtype=torch.int16, device="cuda")
        self._setup(tok, sizes, starts, levels, level_shards, topk, lib, [None] * len(sizes))
        self.copy_stream = torch.cuda.Stream()
        self.queue: list = []

    @classmethod
    def from_device(cls, tok: torch.Tensor, sizes: list[int], starts: list[int], levels=LEVELS, level_shards=None,
                    topk: int = 0, lib: Lib | None = None) -> "CountBuild":
        """A build over shards already laid out in GPU memory (`tok` int16 [L], data.pack_layout's starts)."""
        self = cls.__new__(cls)
        self.rank, self.world, self.host, self.queue = 0, 1, [], []
        self._setup(tok, sizes, starts, levels, level_shards, topk, lib, None)
        return self

    def _setup(self, tok, sizes, starts, levels, level_shards, topk, lib, ready) -> None:
        self.tok, self.sizes, self.starts, self.L = tok, list(sizes), list(starts), int(tok.numel())
        self.levels, self.topk = tuple(levels), topk
        self.lib = lib or Lib()
        self.ready = ready
        self.engine = LevelBuild(tok, sizes, starts, levels, LEVEL_SHARDS if level_shards is None else level_shards,
                                 ready=ready, elib=self.lib)
        self.level_shards = self.engine.level_shards
        self.timing: dict[str, float] = {}
        self.info: dict = {}
        self.load_start = None

    @property
    def kernel_events(self) -> list:
        return self.engine.kernel_events

    def prepare(self) -> None:
        """Before the clock (the reference connects its collectives here; one GPU has none)."""
        torch.cuda.synchronize()

    def start_load(self, steps: int = 1) -> None:
        """The shards' copies (COPY_TOKENS each) split into `steps` shares, the first one enqueued (build.py:231-243)."""
        if not self.host:
            raise ValueError("a build from device tokens has nothing to load")
        self.queue = [(i, a, min(a + COPY_TOKENS, h.numel()))
                      for i, h in enumerate(self.host) for a in range(0, max(h.numel(), 1), COPY_TOKENS)]
        self.share = -(-len(self.queue) // max(1, steps))
        self.ready[:] = [None] * len(self.host)
        # the copies follow whatever the caller's stream did to the buffer (its SENT fill, a refill between builds)
        self.copy_stream.wait_stream(torch.cuda.current_stream())
        self.load_start = torch.cuda.Event(enable_timing=True)
        self.load_start.record(self.copy_stream)
        self.pace()

    def pace(self) -> None:
        """The next share of the copies; a shard's event is recorded after its last copy (build.py:245-255)."""
        batch, self.queue = self.queue[: self.share], self.queue[self.share :]
        with torch.cuda.stream(self.copy_stream):
            for i, a, b in batch:
                at = self.starts[i] + a
                self.tok[at : at + b - a].copy_(self.host[i][a:b], non_blocking=True)
                if b >= self.host[i].numel():
                    ev = torch.cuda.Event(enable_timing=True)
                    ev.record(self.copy_stream)
                    self.ready[i] = ev

    def load_ms(self) -> float:
        """The copies' device time from start_load to the last shard's copy, once all are enqueued (build.py:257-259)."""
        if self.queue or self.load_start is None or any(e is None for e in self.ready):
            raise ValueError("the loads have not all been enqueued")
        last = self.ready[-1]
        last.synchronize()
        return self.load_start.elapsed_time(last)

    def counts(self, x: torch.Tensor, tgt: torch.Tensor, avail: torch.Tensor, stats: bool = False) -> torch.Tensor:
        """int32 [3, len(levels), N] (see the module docstring); `stats`: also each level's corpus hits in self.info."""
        if self.ready is not None and any(e is None for e in self.ready):
            raise ValueError("start_load() first: some shards have no copy enqueued")
        rows = all(k in self.levels for k in ROW_LEVELS)
        res = self.engine.build(x, tgt, avail, topk=self.topk, keep=ROW_LEVELS if rows else (), stats=stats)
        self.info = res.info
        if self.topk:
            self.top_tok, self.top_cnt = res.top_tok, res.top_cnt
        if rows:
            desc = []
            for k in ROW_LEVELS:
                ctx_of, rec = res.kept[k]
                desc += [res.counts[0, self.levels.index(k)].data_ptr(), ctx_of.data_ptr(), rec.data_ptr()]
            d = torch.tensor(desc, dtype=torch.int64, device=x.device)
            N = x.numel()
            self.row_cells = torch.empty(N, dtype=torch.int32, device=x.device)
            self.row_entries = torch.empty((N, ROW_K), dtype=torch.int32, device=x.device)
            self.lib("ng_record_rows", N, i32(len(ROW_LEVELS)), d, self.row_cells, self.row_entries)
            self._keep = (d, res.kept)  # the descriptor's buffers until the kernel has read them
        self.out = res.counts
        return res.counts

    def batch_rows(self, at: int, n: int, capacity: int) -> torch.Tensor:
        """The rows of the n query positions from `at`: their cells, then `capacity` entries (position, token | weight
        << 16) of the non-zero candidates in position order, padded with (i % n, 0) (build.py:390-403). AssertionError
        if the candidates do not fit."""
        cells = self.row_cells[at : at + n]
        entries = self.row_entries[at : at + n]
        n = cells.numel()
        rows = torch.empty(n + 2 * capacity, dtype=torch.int32, device=cells.device)
        work = torch.empty(self.lib.size("ng_batch_rows_work", n), dtype=torch.int32, device=cells.device)
        total = torch.zeros(1, dtype=torch.int64, device=cells.device)
        self.lib("ng_batch_rows", cells, entries, n, capacity, rows, work, total)
        m = int(total.item())
        if m > capacity:
            raise AssertionError(f"{m} candidates overflow the rows' {capacity} entries")
        return rows

