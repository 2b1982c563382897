"""Host driver of the validation-side n-gram statistics on one MI355X: the mirror of old_records/gpu_val_stats.py
(`ValIndex` :604-651, `Scanner` :473-532, `_run` :701-1232, `InProcess` :1235-1316, the CLI :657-685) on our HIP
library, with the same constants, definitions, output layout and error behaviour. One process per GPU; this build runs
one GPU (world 1), so the owner exchange is the identity (the reference's world == 1 path: `recv = send`, no
reduce_by_key, :1020-1022, :1032-1041).

Per level k (ascending): the query index (distinct valid query k-contexts, a canonical linear-probing table, a
representative position each), the scan of every corpus position whose previous level matched (a bitmap), counting
(context id, next token) in a pair table (directly, or emitted and grouped into L2-sized sub-tables), then the
owner's sort, segments, totals, ranks, top-8, and per query position tot / dist / cnt (the target's count if among
the TOP = 1024 most frequent) and the mask bit; then each variant's hint rows from the per-level tops.

Outputs: `counts` int32 [3, len(ALL_LEVELS), N] (tot, dist, cnt; tot and cnt as uint32 bits) and `rows` int32
[len(variants), N, 9] (cell, 4 x two tokens, 4 x two weights), as InProcess.finish() returns; the CLI saves
tot/dist/cnt.npy [N, 10] and rows_<levels>/{cell,tokens,weights}.npy (:1216-1228)."""

from __future__ import annotations

import argparse
import json
import os
import threading
import time
from pathlib import Path

import numpy as np
import torch

from .data import BOS, HEADER_BYTES, shard_tokens
from .lib import Lib, i32, u64
from .loader import Loader

ALL_LEVELS = (2, 3, 4, 5, 6, 8, 10, 12, 16, 20)
LEVELS = (2, 3, 4, 5, 6, 10, 20)  # the hint rows' levels and length buckets
VARIANTS = ((6, 10, 20), (2, 3, 6, 10, 20), LEVELS)
VAL_TOKENS = 10_485_760
GAP = 32  # SENT tokens before each shard (>= the longest context)
TOP = 1024
ENTRIES = 8
# Distinct (context, next) pairs of n training tokens per level (the reference's fit, :93-97), to size pair tables;
# a table that overflows doubles and its level reruns.
PAIRS = {2: (82.17e6, 0.620), 3: (62.30e6, 0.667), 4: (26.39e6, 0.694), 5: (8.99e6, 0.706), 6: (3.17e6, 0.705),
         8: (0.550e6, 0.671), 10: (0.223e6, 0.604), 12: (0.162e6, 0.577), 16: (0.121e6, 0.572), 20: (0.102e6, 0.581)}
SAFETY = 1.15
LOAD = 0.7
SUB_SLOTS = 1 << 16
MAX_PBITS = 12
SIGN = -(1 << 63)


def pairs_estimate(k: int, n_tokens: int) -> float:
    u, beta = PAIRS.get(k, (0.102e6, 0.581))
    return SAFETY * u * (n_tokens / 4e8) ** beta


class Clock:
    """Phase timings: each phase ends with a device synchronize (world 1: no barrier)."""

    def __init__(self):
        self.t = time.time()
        self.phases: list[tuple[str, float, float]] = []

    def lap(self, name: str) -> float:
        torch.cuda.synchronize()
        now = time.time()
        self.phases.append((name, now - self.t, 0.0))
        self.t = now
        return 0.0


def layout(sizes: list[int]) -> tuple[list[int], int]:
    """Each shard's first position (32-aligned, >= GAP after the previous shard) and the buffer length (:391-398)."""
    starts, at = [], GAP
    for n in sizes:
        starts.append(at)
        at = (at + n + GAP + 31) // 32 * 32
    return starts, at


def load_shards(shards: list, device="cuda") -> tuple[torch.Tensor, list[int], list[int], int]:
    """The shards (paths of shard files, or uint16 arrays) in one GPU buffer with SENT gaps: (tok int16 [L], sizes,
    starts, L). Synchronous (the reference's threaded loader overlaps the copies with the index build)."""
    arrays = []
    for s in shards:
        if isinstance(s, (str, os.PathLike)):
            n = shard_tokens(s)
            arrays.append(np.fromfile(s, dtype="<u2", count=n, offset=HEADER_BYTES))
        else:
            arrays.append(np.asarray(s, dtype=np.uint16))
    sizes = [len(a) for a in arrays]
    starts, L = layout(sizes)
    tok = torch.full((L,), -1, dtype=torch.int16, device=device)
    for a, st in zip(arrays, starts):
        if len(a):
            tok[st : st + len(a)].copy_(torch.from_numpy(a.view(np.int16)))
    return tok, sizes, starts, L


def query_tensors(val: np.ndarray, n: int | None = None, device="cuda"):
    """x, tgt, avail of a query stream (its positions' inputs, then one more token: the last target) (:785-793)."""
    val = np.asarray(val, dtype=np.uint16)
    N = len(val) - 1 if n is None else min(n, len(val) - 1)
    x = torch.from_numpy(val[:N].view(np.int16).copy()).to(device)
    tgt = torch.from_numpy(val[1 : N + 1].view(np.int16).copy()).to(device)
    idx = torch.arange(N, device=device, dtype=torch.int64)
    xi = x.to(torch.int32) & 0xFFFF
    seg = torch.cummax(torch.where(xi == BOS, idx, torch.zeros_like(idx)), 0).values
    avail = (idx - seg + 1).to(torch.int32)
    return x, tgt, avail


class ValIndex:
    """One level's query contexts: per position its context id (-1 where invalid), the number of contexts, and the
    lookup table (8-byte slots, a context's id is its slot) with each slot's representative position (:604-651). The
    keys are sorted (unsigned: the order of their home slots) by our radix sort."""

    def __init__(self, lib: Lib, x: torch.Tensor, avail: torch.Tensor, k: int, max_ids: int = (1 << 24) - 4096):
        n = x.numel()
        keys = torch.empty(n, dtype=torch.int64, device=x.device)
        lib("val_keys", x, avail, n, i32(k), keys)
        pos = (keys != -1).nonzero().squeeze(1)
        m = int(pos.numel())
        kv = keys[pos].contiguous()
        pv = pos.to(torch.int32)
        del keys
        sk = torch.empty_like(kv)
        sp = torch.empty_like(pv)
        if m:
            lib.cub("sort_pairs", kv, sk, pv, sp, m, i32(0), i32(64))
        del kv, pv
        spos = sp.long()
        del sp, pos
        new = torch.ones_like(sk, dtype=torch.bool)
        new[1:] = sk[1:] != sk[:-1]
        gid = torch.cumsum(new, 0) - 1
        rep = spos[new].contiguous()
        ukeys = sk[new].contiguous()
        del sk
        self.n = int(ukeys.numel())
        if bool((ukeys == -2).any()):
            raise RuntimeError(f"k={k}: a validation key collides with the empty marker")
        bad = torch.zeros(1, dtype=torch.int64, device=x.device)
        lib("val_verify", x, spos, gid, rep, int(spos.numel()), i32(k), bad)
        if int(bad.item()):
            raise RuntimeError(f"k={k}: {int(bad.item())} validation positions collide with another context's key")
        self.valid = int(spos.numel())
        self.cap = min(2 * self.n + 1024, max_ids)
        home = torch.empty(self.n, dtype=torch.int64, device=x.device)
        lib("val_homes", ukeys, self.n, u64(self.cap), home)
        at = torch.arange(self.n, device=x.device, dtype=torch.int64)
        slot_of = torch.empty_like(home)
        if self.n:
            lib.cub("inclusive_max", home - at, slot_of, self.n)
        slot_of += at
        size = max(self.cap, int(slot_of[-1].item()) + 1 if self.n else 0) + 1
        if size >= max_ids + 4096:
            raise RuntimeError(f"k={k}: {self.n} contexts do not fit {max_ids.bit_length()}-bit ids")
        self.table = torch.full((size,), -1, dtype=torch.int64, device=x.device)
        self.table[slot_of] = ukeys
        self.rep = torch.zeros(size, dtype=torch.int32, device=x.device)
        self.rep[slot_of] = rep.to(torch.int32)
        self.ids = size
        del home, at
        self.ctx_of = torch.full((n,), -1, dtype=torch.int32, device=x.device)
        self.ctx_of[spos] = slot_of[gid].to(torch.int32)


class Scanner:
    """One level's scan over position ranges (each a multiple of 32 positions from a 32-aligned start): counted
    directly in the pair table, or (partitioned) the hits' pair keys emitted into a buffer of up to `chunk` keys, then
    grouped by sub-table and counted sub-table by sub-table (:473-532)."""

    def __init__(self, lib, k, vi, x, tok, bm_prev, bm_next, table, grid, partitioned, sparse, chunk, pbits):
        self.lib, self.k, self.vi, self.x, self.tok = lib, k, vi, x, tok
        self.bm_prev, self.bm_next, self.table, self.grid = bm_prev, bm_next, table, grid
        self.partitioned, self.sparse, self.chunk, self.pbits = partitioned, sparse, chunk, pbits
        self.words = False
        self.times: dict[str, float] = {}
        self.events: list = []
        self.pending = 0
        if partitioned:
            self.emit = torch.empty(chunk, dtype=torch.int64, device="cuda")
            self.grouped = torch.empty(chunk, dtype=torch.int64, device="cuda")
            self.emitted = torch.zeros(1, dtype=torch.int64, device="cuda")
            self.counts = torch.zeros(1 << pbits, dtype=torch.int64, device="cuda")

    def scan(self, start: int, n: int) -> None:
        if self.partitioned and self.pending + n > self.chunk:
            self.flush()
        bm_in = None if self.bm_prev is None else self.bm_prev[start // 32 :]
        if self.partitioned:
            mode = 3 if bm_in is not None and self.words else 2
        else:
            mode = int(self.sparse and bm_in is not None)
        pk, pc, sub_cap, pbits, flags = self.table
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        self.lib("scan_level", self.tok[start:], n, i32(self.k), bm_in, self.bm_next[start // 32 :], self.vi.table,
                 u64(self.vi.cap), self.vi.rep, self.x, pk, pc, sub_cap, pbits, flags, i32(self.grid), i32(mode),
                 self.emit if self.partitioned else None, self.emitted if self.partitioned else None)
        e1.record()
        self.events.append(("scan", e0, e1))
        self.pending += n

    def flush(self) -> None:
        if not self.partitioned or self.pending == 0:
            return
        torch.cuda.current_stream().synchronize()
        t0 = time.time()
        n = int(self.emitted.item())
        pk, pc, sub_cap, pbits, flags = self.table
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record()
        self.counts.zero_()
        self.lib("subpart_count", self.emit, n, pbits, self.counts)
        cursor = torch.cumsum(self.counts, 0) - self.counts
        self.lib("subpart_scatter", self.emit, n, pbits, cursor, self.grouped)
        e[1].record()
        self.lib("aggregate", self.grouped, n, pk, pc, sub_cap, pbits, flags, i32(self.grid))
        e[2].record()
        torch.cuda.current_stream().synchronize()
        self.events += [("group", e[0], e[1]), ("aggregate", e[1], e[2])]
        self.times["flush_wall"] = self.times.get("flush_wall", 0.0) + time.time() - t0
        self.emitted.zero_()
        self.pending = 0


def parse_args(argv: list[str] | None = None) -> argparse.Namespace:
    """The reference's flags (:657-681); the multi-GPU and I/O ones are accepted and have no effect on one GPU."""
    ap = argparse.ArgumentParser()
    ap.add_argument("--shards", required=True, help="a file listing the training shard paths")
    ap.add_argument("--val", required=True, help="the validation shard")
    ap.add_argument("--out", required=True)
    ap.add_argument("--threads", type=int, default=8)
    ap.add_argument("--load-mode", choices=("register", "pread"), default="pread")
    ap.add_argument("--chunk-mb", type=int, default=16)
    ap.add_argument("--sequential", action="store_true")
    ap.add_argument("--direct", action="store_true", help="count every level directly in its pair table")
    ap.add_argument("--pipeline", action="store_true")
    ap.add_argument("--async-init", action="store_true")
    ap.add_argument("--nccl-warmup", action="store_true")
    ap.add_argument("--own-device", action="store_true")
    ap.add_argument("--ipc", action="store_true")
    ap.add_argument("--early-ctx", action="store_true")
    ap.add_argument("--fused", action="store_true", help="scan each shard through every level (direct)")
    ap.add_argument("--numa", action="store_true")
    ap.add_argument("--words-density", type=float, default=0.0)
    ap.add_argument("--chunk-positions", type=int, default=0)
    ap.add_argument("--bench-io", action="store_true")
    ap.add_argument("--no-save", action="store_true")
    ap.add_argument("--val-tokens", type=int, default=VAL_TOKENS)
    ap.add_argument("--launch-time", type=float, default=float("nan"))
    return ap.parse_args(argv)


def build_stats(lib: Lib, tok: torch.Tensor, L: int, starts: list[int], sizes: list[int], x: torch.Tensor,
                tgt: torch.Tensor, avail: torch.Tensor, *, levels=ALL_LEVELS, variants=VARIANTS, direct=False,
                fused=False, words_density=0.0, chunk_positions=0, sub_slots=SUB_SLOTS, max_pbits: int | None = None,
                grid: int | None = None, min_cap: int = 1 << 20, loader=None) -> dict:
    """The whole build on one GPU from resident tokens and queries (the body of _run :784-1152 with world 1).
    `loader`: a started Loader still copying the shards into `tok`: the query index is built meanwhile, and each
    shard's first scan waits for that shard's copy only (:877, :959). Returns {"counts", "rows", "levels", "timing"}."""
    N = x.numel()
    n_tokens = sum(sizes)
    clock = Clock()
    timing: dict = {}
    props = torch.cuda.get_device_properties(tok.device)
    if grid is None:
        grid = props.multi_processor_count * 32
    mp = min(max_pbits or MAX_PBITS, lib.plain("max_pbits"))
    index = {k: ValIndex(lib, x, avail, k) for k in levels}
    clock.lap("val_index")
    timing["val_index"] = {k: {"contexts": v.n, "valid": v.valid} for k, v in index.items()}
    out_cnts = torch.zeros((3, len(levels), N), dtype=torch.int32, device=tok.device)
    mask = torch.zeros(N, dtype=torch.int32, device=tok.device)
    tops: dict = {}
    nwords = L // 32
    bm_prev = None
    bm_next = torch.empty(nwords, dtype=torch.int32, device=tok.device)
    popc = torch.zeros(1, dtype=torch.int64, device=tok.device)
    levels_info: dict = {}
    free = torch.cuda.mem_get_info()[0] + torch.cuda.memory_reserved() - torch.cuda.memory_allocated()
    chunk = chunk_positions or min(1 << 29, int(free * 0.15 / 16))
    chunk = max(1 << 20, chunk // 32 * 32)
    fused_tables: dict = {}
    if fused:
        for k in levels:
            cap = max(1 << 20, int(min(pairs_estimate(k, n_tokens), n_tokens) / LOAD))
            fused_tables[k] = (torch.full((cap,), -1, dtype=torch.int64, device=tok.device),
                               torch.zeros((cap + 3) // 4, dtype=torch.int32, device=tok.device), cap,
                               torch.zeros(2, dtype=torch.int32, device=tok.device))
        bms = [bm_next, torch.zeros(nwords, dtype=torch.int32, device=tok.device)]
        bms[0].zero_()
        for i, (st, n) in enumerate(zip(starts, sizes)):
            if loader is not None:
                torch.cuda.current_stream().wait_event(loader.wait(i))
            n32 = (n + 31) // 32 * 32
            for li, k in enumerate(levels):
                vi = index[k]
                pk, pc, cap, flags = fused_tables[k]
                bm_in = None if li == 0 else bms[(li - 1) % 2][st // 32 :]
                mode = 0 if li == 0 or k <= 5 else 1
                lib("scan_level", tok[st:], n32, i32(k), bm_in, bms[li % 2][st // 32 :], vi.table, u64(vi.cap),
                    vi.rep, x, pk, pc, u64(cap), i32(0), flags, i32(grid), i32(mode), None, None)
        torch.cuda.synchronize()
        bad = [k for k in levels if int(fused_tables[k][3][0].item())]
        if bad:
            raise RuntimeError(f"fused scan: the pair tables of levels {bad} overflowed")
        del bms
        clock.lap("scan_all")
    for li, k in enumerate(levels):
        info: dict = {}
        vi = index[k]
        bounds = torch.tensor([0, vi.ids], dtype=torch.int64, device=tok.device)
        lo, hi = 0, vi.ids
        if fused:
            pk, pc, cap, flags = fused_tables.pop(k)
            fl = flags.cpu().tolist()
            info.update(contexts=vi.n, cap=cap, false_hash_hits=fl[1], fused=True)
        else:
            if bm_prev is None:
                active = n_tokens
            else:
                popc.zero_()
                lib("popcount", bm_prev, nwords, popc)
                active = int(popc.item())
            free = torch.cuda.mem_get_info()[0] + torch.cuda.memory_reserved() - torch.cuda.memory_allocated()
            est = min(pairs_estimate(k, n_tokens), active)
            cap = max(min_cap, int(est / LOAD))
            cap = min(cap, int(free * 0.45 / 9))
            sparse = bm_prev is not None and active * 16 < L
            partitioned = not sparse and cap > 4 * sub_slots and not direct
            reruns = 0
            while True:
                pbits = min(mp, max(1, (cap // sub_slots).bit_length())) if partitioned else 0
                sub_cap = -(-cap // (1 << pbits))
                cap = sub_cap << pbits
                pk = torch.full((cap,), -1, dtype=torch.int64, device=tok.device)
                pc = torch.zeros((cap + 3) // 4, dtype=torch.int32, device=tok.device)
                flags = torch.zeros(2, dtype=torch.int32, device=tok.device)
                table = (pk, pc, u64(sub_cap), i32(pbits), flags)
                first = bm_prev is None
                if first:
                    bm_next.zero_()
                    ranges = [(st, (n + 31) // 32 * 32) for st, n in zip(starts, sizes)]
                else:
                    ranges = [(0, L)]
                scanner = Scanner(lib, k, vi, x, tok, bm_prev, bm_next, table, grid, partitioned, sparse, chunk, pbits)
                scanner.words = active * words_density < L if words_density > 0 else False
                for i, (st, n) in enumerate(ranges):
                    if first and loader is not None:
                        torch.cuda.current_stream().wait_event(loader.wait(i))
                    for a in range(0, n, chunk):
                        scanner.scan(st + a, min(n, a + chunk) - a)
                scanner.flush()
                torch.cuda.current_stream().synchronize()
                fl = flags.cpu().tolist()
                if fl[0] == 0:
                    break
                reruns += 1
                del pk, pc, scanner
                cap *= 2
            for name, e0, e1 in scanner.events:
                scanner.times[name] = scanner.times.get(name, 0.0) + e0.elapsed_time(e1) / 1e3
            info["scan_parts_s"] = scanner.times
            del scanner
            popc.zero_()
            lib("popcount", bm_next, nwords, popc)
            hits = int(popc.item())
            clock.lap(f"k{k}.scan")
            info.update(contexts=vi.n, active=active, hits=hits, cap=cap, reruns=reruns, sparse=sparse, pbits=pbits,
                        sub_cap=sub_cap, partitioned=partitioned, false_hash_hits=fl[1])
        # local aggregation (world 1: every entry is this rank's), sort, segments, totals, ranks, outputs
        counts = torch.zeros(1, dtype=torch.int64, device=tok.device)
        lib("part_count", pk, u64(cap), bounds, i32(1), counts)
        u_local = int(counts.item())
        cursor = torch.zeros(1, dtype=torch.int64, device=tok.device)
        send_k = torch.empty(u_local, dtype=torch.int64, device=tok.device)
        send_c = torch.empty(u_local, dtype=torch.int32, device=tok.device)
        lib("part_scatter", pk, pc, u64(cap), bounds, i32(1), cursor, send_k, send_c)
        del pk, pc
        n_own = hi - lo
        ctx_bits = max(1, (max(n_own, 2) - 1).bit_length())
        sk = torch.empty_like(send_k)
        sc = torch.empty_like(send_c)
        if u_local:
            lib.cub("sort_pairs", send_k, sk, send_c, sc, u_local, i32(0), i32(16 + ctx_bits))
        del send_k, send_c
        uk, agg, U = sk, sc, u_local
        start = torch.zeros(n_own, dtype=torch.int64, device=tok.device)
        end = torch.zeros(n_own, dtype=torch.int64, device=tok.device)
        lib("seg_bounds", uk, U, start, end)
        tot = torch.empty(n_own, dtype=torch.int64, device=tok.device)
        lib("ctx_tot", start, end, agg, n_own, tot)
        key2 = torch.empty(U, dtype=torch.int64, device=tok.device)
        val2 = torch.empty(U, dtype=torch.int32, device=tok.device)
        lib("rank_keys", uk, agg, U, key2, val2)
        k2s = torch.empty_like(key2)
        sv = torch.empty_like(val2)
        if U:
            lib.cub("sort_pairs", key2, k2s, val2, sv, U, i32(0), i32(32 + ctx_bits))
        del key2, val2, k2s
        rank_of = torch.empty(U, dtype=torch.int32, device=tok.device)
        top_tok = top_cnt = None
        if k in LEVELS:
            top_tok = torch.zeros(n_own * ENTRIES, dtype=torch.int16, device=tok.device)
            top_cnt = torch.zeros(n_own * ENTRIES, dtype=torch.int32, device=tok.device)
        lib("rank_scatter", sv, U, uk, agg, start, rank_of, top_tok, top_cnt, i32(ENTRIES))
        del sv
        lib("pos_outputs", vi.ctx_of, N, lo, hi, tgt, uk, agg, rank_of, start, end, tot, i32(li), i32(TOP),
            out_cnts[0, li], out_cnts[1, li], out_cnts[2, li], mask)
        max_tot = int(tot.max().item()) if n_own else 0
        if max_tot >= 1 << 32:
            raise RuntimeError(f"k={k}: a total of {max_tot} does not fit uint32")
        if k in LEVELS:
            tops[k] = (top_tok, top_cnt, tot, lo, hi)
        del uk, agg, rank_of, start, end
        clock.lap(f"k{k}.rows")
        info.update(owned=n_own, pairs_local=u_local, pairs_owned=U)
        levels_info[k] = info
        if not fused:
            bm_prev, bm_next = bm_next, (bm_prev if bm_prev is not None else
                                         torch.empty(nwords, dtype=torch.int32, device=tok.device))
    rows = torch.zeros((len(variants), N, 9), dtype=torch.int32, device=tok.device)
    for v, lv in enumerate(variants):
        desc = []
        for k in lv:
            top_tok, top_cnt, tot, lo, hi = tops[k]
            desc += [levels.index(k), LEVELS.index(k), index[k].ctx_of.data_ptr(), lo, hi, top_tok.data_ptr(),
                     top_cnt.data_ptr(), tot.data_ptr()]
        desc_t = torch.tensor(desc, dtype=torch.int64, device=tok.device)
        lib("variant_rows", N, mask, i32(len(lv)), desc_t, rows[v])
        torch.cuda.synchronize()  # desc_t's pointers stay valid until the kernel ran
    clock.lap("rows")
    timing["phases"] = clock.phases
    return {"counts": out_cnts, "rows": rows, "levels": levels_info, "timing": timing, "mask": mask}


def host_outputs(result: dict, variants=VARIANTS) -> dict[str, np.ndarray]:
    """The CLI's output arrays (:1173-1180): tot/dist/cnt [N, L], cell [V, N], tokens/weights [V, N, 8]."""
    c, rows = result["counts"], result["rows"]
    return {
        "tot": c[0].t().contiguous().cpu().numpy().view(np.uint32),
        "dist": c[1].t().to(torch.int16).contiguous().cpu().numpy().view(np.uint16),
        "cnt": c[2].t().contiguous().cpu().numpy().view(np.uint32),
        "cell": rows[:, :, 0].to(torch.int16).contiguous().cpu().numpy(),
        "tokens": rows[:, :, 1:5].contiguous().view(torch.int16).cpu().numpy().view(np.uint16),
        "weights": rows[:, :, 5:9].contiguous().view(torch.int16).cpu().numpy().view(np.uint16),
    }


def run(args: argparse.Namespace) -> dict:
    """main()'s build: shards and validation from files, outputs to args.out (world 1)."""
    t0 = time.time()
    torch.cuda.set_device(0)
    lib = Lib()
    paths = [p for p in Path(args.shards).read_text().split() if p]
    sizes = [shard_tokens(p) for p in paths]
    starts, L = layout(sizes)
    loader = Loader(paths, L, starts, sizes, args.threads, args.load_mode, args.chunk_mb << 19, args.numa)
    n_val = shard_tokens(args.val)
    val = np.fromfile(args.val, dtype="<u2", count=min(n_val, args.val_tokens + 1), offset=HEADER_BYTES)
    x, tgt, avail = query_tensors(val, args.val_tokens)
    res = build_stats(lib, loader.tok, L, starts, sizes, x, tgt, avail, direct=args.direct, fused=args.fused,
                      words_density=args.words_density, chunk_positions=args.chunk_positions, loader=loader)
    loader.join()
    torch.cuda.synchronize()
    res["timing"]["total_s"] = time.time() - t0
    res["timing"]["load"] = {"seconds": loader.stats["seconds"], "bytes": loader.stats["bytes"],
                             "threads": args.threads}
    out = Path(args.out)
    if not args.no_save:
        out.mkdir(parents=True, exist_ok=True)
        host = host_outputs(res)
        for name in ("tot", "dist", "cnt"):
            np.save(out / f"{name}.npy", host[name])
        for v, levels in enumerate(VARIANTS):
            d = out / f"rows_{'_'.join(map(str, levels))}"
            d.mkdir(exist_ok=True)
            np.save(d / "cell.npy", host["cell"][v])
            np.save(d / "tokens.npy", host["tokens"][v])
            np.save(d / "weights.npy", host["weights"][v])
        (out / "timings.json").write_text(json.dumps([res["timing"]], indent=1, default=str))
    return res


def main() -> None:
    run(parse_args())


class InProcess:
    """The build inside a process that holds the GPU (InProcess of :1235-1316), one GPU:
      - construct (before the clock): the shards' layout, the GPU token buffer and the loader's pinned staging buffers
        allocated, the library loaded;
      - prepare() (before the clock): nothing to connect on one GPU;
      - start_load() (optional, on the clock): the shard loads start in background threads while the caller runs;
      - start_background() (optional, instead of start_load): the loads and the whole build on a background thread
        and a HIP stream of their own (one GPU has no collectives, so nothing has to wait for finish());
      - finish(): waits for the loads (starting them if nothing did), builds the query index while the last shards
        land, scans each shard once its copy is done, then the merges and rows -> {"counts": int32
        [3, len(ALL_LEVELS), N] (tot, dist, cnt; tot and cnt as uint32 bits), "rows": int32 [len(variants), N, 9],
        "timing"}.
    `variants`: the hint rows' level sets (each of LEVELS)."""

    def __init__(self, shard_paths: list[str], val_path: str, variants=(LEVELS,), threads: int = 12, chunk_mb: int = 16,
                 flags: tuple[str, ...] = ("--fused", "--direct"), val_tokens: int = VAL_TOKENS):
        self.variants = tuple(tuple(v) for v in variants)
        if not all(set(v) <= set(LEVELS) for v in self.variants):
            raise ValueError(f"variants {self.variants} must be of {LEVELS}")
        self.args = parse_args(["--shards", "-", "--val", val_path, "--out", "-", "--threads", str(threads),
                                "--chunk-mb", str(chunk_mb), "--val-tokens", str(val_tokens), *flags])
        self.paths = list(shard_paths)
        self.sizes = [shard_tokens(p) for p in self.paths]
        self.starts, self.L = layout(self.sizes)
        self.device = torch.cuda.current_device()
        self.loader = Loader(self.paths, self.L, self.starts, self.sizes, threads, "pread", chunk_mb << 19, start=False)
        self.loader.preallocate()
        self.lib = Lib()
        self.thread, self.error, self.result = None, None, None

    def prepare(self) -> None:
        torch.cuda.synchronize()

    def start_load(self) -> None:
        if not self.loader.started:
            self.loader.start()

    def start_background(self) -> None:
        """The loads and the build from now, on a background thread and stream; finish() returns its result."""
        if self.thread is not None:
            raise ValueError("the build has already started")
        self.start_load()
        stream = torch.cuda.Stream(device=self.device)

        def work() -> None:
            try:
                torch.cuda.set_device(self.device)
                with torch.cuda.stream(stream):
                    self.result = self._build()
                stream.synchronize()
            except BaseException as e:  # noqa: BLE001 - raised again by finish()
                self.error = e

        self.thread = threading.Thread(target=work, daemon=True)
        self.thread.start()

    def _build(self) -> dict:
        t0 = time.time()
        n_val = shard_tokens(self.args.val)
        val = np.fromfile(self.args.val, dtype="<u2", count=min(n_val, self.args.val_tokens + 1), offset=HEADER_BYTES)
        x, tgt, avail = query_tensors(val, self.args.val_tokens)
        res = build_stats(self.lib, self.loader.tok, self.L, self.starts, self.sizes, x, tgt, avail,
                          variants=self.variants, direct=self.args.direct, fused=self.args.fused,
                          words_density=self.args.words_density, chunk_positions=self.args.chunk_positions,
                          loader=self.loader)
        self.loader.join()
        res["timing"]["total_s"] = time.time() - t0
        res["timing"]["load"] = {"seconds": self.loader.stats["seconds"], "bytes": self.loader.stats["bytes"]}
        return {"counts": res["counts"], "rows": res["rows"], "timing": res["timing"]}

    def finish(self) -> dict:
        if self.thread is None:
            self.start_load()
            return self._build()
        t0 = time.time()
        self.thread.join()
        self.waited = time.time() - t0
        if self.error is not None:
            raise self.error
        torch.cuda.current_stream().synchronize()
        return self.result


if __name__ == "__main__":
    main()
