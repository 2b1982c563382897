"""The engine's query index (libngram_amd.so ng_query_index): per level, the distinct valid query k-contexts inserted
into an open-addressing table by compare-and-swap, with no sort. The same attributes as gpu_val_stats.ValIndex
(`n`, `valid`, `cap`, `table`, `rep`, `ids`, `ctx_of`), so the engine's scans probe it the same way (linear probing
without wrap-around from umulhi(key, cap); the table ends with an empty slot). Unlike ValIndex's canonical, sorted
layout (the reference's, gpu_val_stats.py:604-651, which makes ids agree across ranks), slots follow insertion races;
on one GPU every output is id-independent, so any layout is exact. Hashed keys (k > 4) are verified against each
slot's representative (the position whose compare-and-swap inserted it): a 64-bit collision raises, as ValIndex's does."""

from __future__ import annotations

import torch

from .lib import Lib, i32, u64

TAIL = 4096  # slots past cap that linear probing may run into; the last stays empty
LOAD = 0.3  # contexts per slot aimed at: at c3 with the scans' two-slot lookups 0.25-0.35 are fastest (0.4 +2%,
# 0.5 +7%, 0.6 +16% per step): a shorter walk matters more than a smaller table
SHRINK = 2.0  # a table more than this many times the size its contexts need moves to one of that size
EXPECT_MARGIN = 1.2  # a table sized from an expected context count holds this many times it at LOAD (1 at least)


class QueryIndex:
    def __init__(self, lib: Lib, x: torch.Tensor, avail: torch.Tensor, k: int, positions: torch.Tensor | None = None,
                 compact: bool = False, expect: int | None = None, _resized: bool = False, defer: bool = False,
                 n_dev: torch.Tensor | None = None, counters: torch.Tensor | None = None, load: float | None = None):
        """Index the valid k-contexts of the query positions (all of x, or the int32 `positions`). `compact`: ctx_of
        holds one entry per listed position (in their order) instead of one per position of x. `expect`: about how
        many contexts there are (e.g. the last build's count): the table is sized for them at once instead of for
        every position and shrunk; if they turn out more than the table holds at LOAD, the index is built once more,
        sized for the count found (`_resized` marks that second build, which keeps its table whatever its load).
        `defer` (with `expect`): the build's counters are not read here, so the host does not wait for the GPU; the
        table sized from `expect` stands, `n` is None, and the caller must pass `pending` to `check()` and redo its
        work if an insert found no slot (its context is then missing from the table). `n_dev` (int64 [1] on the
        device, with `positions`): only the first n_dev of the listed positions are indexed (a count the host has not
        read; `positions` holds at least that many, or the caller checks). `counters` (int64 [3] of zeros on the device,
        with `defer`): where the deferred build's counters go (e.g. a row of the caller's stats, read with its other
        results in one copy), else new. `load`: the contexts per slot a table sized from a context count aims at (LOAD
        if None); a sparser table shortens the probe walks of a level probed at every position."""
        dev = x.device
        ld = LOAD if load is None else load
        N = x.numel()
        m = N if positions is None else int(positions.numel())
        full = int(m / LOAD) + 1024  # room for every position's context at LOAD
        cap = full
        if expect is not None:
            cap = min(cap, int(max(expect, 1) * max(EXPECT_MARGIN, 1.0) / ld) + 1024)
        while True:
            slots = cap + TAIL
            table = lib.full_ones(slots, torch.int64, dev)
            rep = torch.empty(slots, dtype=torch.int32, device=dev)  # read only at occupied slots: no fill
            if compact and positions is not None:
                ctx_of = torch.empty(m, dtype=torch.int32, device=dev)
            else:
                ctx_of = lib.full_ones(N, torch.int32, dev) if positions is not None else \
                    torch.empty(N, dtype=torch.int32, device=dev)
            if counters is None or not (defer and expect is not None and not _resized):
                counters = lib.zeros(3, torch.int64, dev)
            if m:
                wave_ins = torch.empty((m + 255) // 256 * 4, dtype=torch.int32, device=dev)  # inserts per wave
                lib("ng_query_index", x, avail, positions, m, n_dev, i32(k), table, u64(cap), u64(slots), rep,
                    ctx_of, i32(int(compact and positions is not None)), counters, wave_ins)
            if defer and expect is not None and not _resized:
                self.pending = counters
                self.n, self.cap, self.ids, self.table, self.rep, self.ctx_of = None, cap, slots, table, rep, ctx_of
                self._valid = None
                return
            c = counters.cpu().tolist()
            if c[1] == 0:
                break
            # an insert walked too far or reached the table's end: a table sized from a wrong estimate moves to the
            # size its positions need; one already that size (never at load <= 1/2 in practice) doubles
            cap = full if cap < full else cap * 2
        if c[2]:
            raise RuntimeError(f"k={k}: {c[2]} query positions collide with another context's key")
        n_ctx = int(c[0])
        if expect is not None and not _resized and n_ctx > ld * cap:  # fuller than aimed at: once more, at their size
            self.__init__(lib, x, avail, k, positions, compact, n_ctx, _resized=True, n_dev=n_dev, load=load)
            return
        if m and cap > SHRINK * (n_ctx / ld) + 4096:
            # sized for every position, used by far fewer contexts: move them to a table sized for them (fewer bits
            # per context id, probes that stay in cache more often)
            small = int(n_ctx / ld) + 1024
            while True:
                t2 = torch.full((small + TAIL,), -1, dtype=torch.int64, device=dev)
                r2 = torch.empty(small + TAIL, dtype=torch.int32, device=dev)
                remap = torch.empty(slots, dtype=torch.int32, device=dev)
                c2 = torch.zeros(3, dtype=torch.int64, device=dev)
                lib("ng_query_index_shrink", table, rep, u64(slots), t2, u64(small), u64(small + TAIL), r2, ctx_of,
                    ctx_of.numel(), remap, c2)
                if int(c2[1].item()) == 0:
                    break
                small *= 2
            table, rep, cap, slots = t2, r2, small, small + TAIL
            del remap
        self.n = n_ctx
        self.cap = cap
        self.ids = slots
        self.table = table
        self.rep = rep
        self.ctx_of = ctx_of
        self._valid = None

    @staticmethod
    def check(pending: list, values: list | None = None) -> list[tuple[int, bool]]:
        """Deferred builds' counters ((k, the index's `pending`) pairs, read here in one copy; or `values`, their host
        values the caller read): per index (n contexts, whether every insert found its slot); a 64-bit key collision
        raises."""
        if not pending:
            return []
        got = values if values is not None else torch.stack([c for _, c in pending]).cpu().tolist()
        out = []
        for (k, _), (n, over, coll) in zip(pending, got):
            if coll:
                raise RuntimeError(f"k={k}: {coll} query positions collide with another context's key")
            out.append((int(n), over == 0))
        return out

    @property
    def valid(self) -> int:
        if self._valid is None:
            self._valid = int((self.ctx_of >= 0).sum().item())
        return self._valid
