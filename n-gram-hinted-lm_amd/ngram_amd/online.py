"""Online causal rows under the step rule on one MI355X, behind exact_match's OnlineRows surface
(exact_match/exact_match.pyi :120-171; exact_match/src/online.rs): a run's training stream (`tokens` in parts
`bounds`), when each position is trained (`spans` [m, 3]: (lo, hi, step), inputs [lo, hi) of `step`, hi its last
target), and per step the hint rows (train_hints.rs's: the deepest of `levels` whose context has a counted
occurrence; its cell, `entries` next tokens and weights) and count rows (train_counts.rs's: tot, dist, cnt of the own
next token) of the queries trained in that step. An occurrence (k tokens within a part and the token after them)
counts for a step-s query iff all its k + 1 tokens were trained before s (alpha = 1 + max tau <= s, online.rs:11-13);
a query's k-context must lie in its segment (segments start at each part's start and at every BOS).

`advance(step_hi, ...)` is the incremental path (online.rs :333): the GPU state (per level a context table with
totals, distinct counts and exact top-`entries` lists, and a split pair table) persists between calls; a step inserts
its newly available occurrences, then answers its queries (libngram_amd.so: ng_online_insert_levels, sort_pairs,
reduce_by_key, ng_online_top, ng_online_query_levels, ng_online_rows). `hints` / `counts` answer a step range from a fresh
state; with rule="segment" (the reference's exactness-test rule) they answer every position from its segment's
start, one step per segment."""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from .data import BOS
from .lib import Lib, i32, u64


MAX_LAUNCH_LEVELS = 8  # levels per fused insert / query launch (ng_online_insert_levels, ng_online_query_levels)
REC_TOP, REC_CNT = 16, 2  # u32 words of a context's record with and without top entries (online.hip OREC_*)


def _ptr(t: torch.Tensor, at: int = 0) -> int:
    """The device address of element `at` of t."""
    return t.data_ptr() + at * t.element_size()


def _i64_array(rows) -> ctypes.Array:
    """Level rows of ints as one host int64 array (values of 2^63 and above wrap, as a u64 argument would)."""
    flat = [v - (1 << 64) if v >= 1 << 63 else v for row in rows for v in row]
    return (ctypes.c_int64 * len(flat))(*flat)

NONE = 0xFFFFFFFF
LOAD = 0.5


def loader_plan(ntok, nproc: int, BT: int, accum: int, steps: int) -> np.ndarray:
    """A training run's plan under llm.c's sequential loader (old_records/r001_llmc_c/llmc/hint_stats.cuh
    loader_plan :395-409): every rank's micro-batches, [m, 5] int64 rows (step, micro, rank, shard, offset), rank r's
    b-th micro-batch the inputs [offset, offset + BT) of its shard; a rank moves to the next shard once a shard's
    (ntok - 1) // (nproc * BT) samples are used. ValueError if the plan runs past the shards."""
    if nproc < 1 or BT < 1 or accum < 1 or steps < 0:
        raise ValueError(f"bad plan: nproc {nproc}, BT {BT}, accum {accum}, steps {steps}")
    plan = []
    for r in range(nproc):
        shard = sample = 0
        for b in range(steps * accum):
            if sample >= (int(ntok[shard]) - 1) // (nproc * BT):
                shard, sample = shard + 1, 0
                if shard >= len(ntok):
                    raise ValueError(f"the training plan runs past the {len(ntok)} shards")
            plan.append((b // accum, b % accum, r, shard, sample * nproc * BT + r * BT))
            sample += 1
    return np.array(plan, np.int64).reshape(-1, 5)


def plan_stream(ntok, plan: np.ndarray, BT: int) -> list[int]:
    """The training stream's parts for a plan (hint_stats.cuh train_plan :666-676): each shard the plan reads, up to
    its last trained target (shard 0 whole)."""
    nshards = int(plan[:, 3].max()) + 1 if len(plan) else 1
    sizes = [0] * nshards
    for _, _, _, shard, off in plan:
        sizes[shard] = max(sizes[shard], int(off) + BT + 1)
    sizes[0] = max(sizes[0], int(ntok[0]))
    return sizes


def plan_spans(plan: np.ndarray, sizes: list[int], BT: int) -> np.ndarray:
    """OnlineRows spans [m, 3] (lo, hi, step) of a plan over the stream of `sizes` parts: every micro-batch's inputs
    [lo, lo + BT) trained in its step, lo + BT its last target (hint_stats.cuh tr_spans_k :411-420)."""
    starts = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    lo = starts[plan[:, 3]] + plan[:, 4]
    return np.stack([lo, lo + BT, plan[:, 0]], axis=1).astype(np.int64)


def plan_rows(plan: np.ndarray, sizes: list[int], BT: int, accum: int, rank: int) -> np.ndarray:
    """The stream position of each of rank `rank`'s training rows, in training order: row (step * accum + micro) * BT
    + i is input i of that micro-batch (hint_stats.cuh's row_of :411-420). Gather a stream-sized output with it."""
    starts = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    mine = plan[plan[:, 2] == rank]
    rows = np.full(int(plan[:, 0].max() + 1) * accum * BT if len(plan) else 0, -1, np.int64)
    for step, micro, _, shard, off in mine:
        r0 = (int(step) * accum + int(micro)) * BT
        rows[r0 : r0 + BT] = starts[shard] + off + np.arange(BT)
    return rows


def _tau(n: int, bounds: list[int], spans: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """tau (first step training a position as an input or a target) and tau_in (as an input) (online.rs:137-158)."""
    tau = np.full(n, NONE, np.uint64)
    tau_in = np.full(n, NONE, np.uint64)
    b = np.asarray(bounds, np.int64)
    sp = np.asarray(spans, np.int64).reshape(-1, 3)
    order = np.argsort(sp[:, 2], kind="stable")[::-1]  # larger steps first: smaller ones overwrite (a minimum)
    for lo, hi, step in sp[order]:
        tau[lo:hi] = np.minimum(tau[lo:hi], step)
        tau_in[lo:hi] = np.minimum(tau_in[lo:hi], step)
        if hi > lo and hi < n:
            part = int(np.searchsorted(b, hi - 1, side="right"))
            if hi < b[part]:
                tau[hi] = min(int(tau[hi]), int(step))
    return tau, tau_in


class OnlineRows:
    """A run's training stream and when each of its positions is trained, for its online hint and count rows under
    the step rule, on the GPU (ValueError on bad tokens, bounds or spans, as online.rs new :118-181)."""

    def __init__(self, tokens, bounds: list[int], spans, threads: int = 1, cpus: list[int] = ()):
        tok = np.ascontiguousarray(tokens, dtype=np.uint16)
        n = len(tok)
        if n == 0 or n >= 1 << 30:
            raise ValueError(f"{n} tokens: need 1 to 2^30")
        bounds = [int(b) for b in bounds]
        if len(bounds) < 2 or bounds[0] != 0 or bounds[-1] != n or any(a >= b for a, b in zip(bounds, bounds[1:])):
            raise ValueError("bounds must ascend strictly from 0 to the token count")
        sp = np.asarray(spans, dtype=np.int64)
        if sp.ndim != 2 or sp.shape[1] != 3:
            raise ValueError("spans must be [m, 3]: (lo, hi, step)")
        if len(sp) and ((sp[:, 0] < 0).any() or (sp[:, 0] > sp[:, 1]).any() or (sp[:, 1] > n).any()
                        or (sp[:, 2] < 0).any() or (sp[:, 2] >= NONE).any()):
            raise ValueError("bad span")
        self.n = n
        self.bounds = bounds
        self.lib = Lib()
        dev = torch.device("cuda", torch.cuda.current_device())
        self.dev = dev
        self.tok = torch.from_numpy(tok.view(np.int16).copy()).to(dev)
        tau, tau_in = _tau(n, bounds, sp)
        self.tau = torch.from_numpy(tau.astype(np.int64)).to(dev)
        self.tau_in = torch.from_numpy(tau_in.astype(np.int64)).to(dev)
        # segments (start at each part and at every BOS), the next token's part, each position's part bounds
        idx = torch.arange(n, device=dev)
        part_of = torch.bucketize(idx, torch.tensor(bounds[1:], device=dev), right=True)
        bt = torch.tensor(bounds, device=dev)
        self.part_lo, self.part_hi = bt[part_of], bt[part_of + 1]
        start = ((self.tok.to(torch.int32) & 0xFFFF) == BOS) | (idx == self.part_lo)
        seg = torch.cummax(torch.where(start, idx, torch.zeros_like(idx)), 0).values
        self.avail = (idx - seg + 1).to(torch.int32)
        self.seg_index = torch.cumsum(start.to(torch.int64), 0) - 1  # the rule "segment"'s steps
        self.has_next = (idx + 1 < self.part_hi).to(torch.uint8)
        self._done = 0
        self.config = None
        self.state = None
        # a step's merge: "buckets" (ng_online_merge: no sort of the step's events, where its packed words hold the
        # step's occurrences) or "sorted" (sort_pairs + reduce_by_key + ng_online_top); both give the same state
        self.merge = "buckets"

    def __len__(self) -> int:
        return self.n

    @property
    def done(self) -> int:
        return self._done

    def prefault(self) -> None:
        torch.cuda.synchronize(self.dev)

    # -----------------------------------------------------------------------------------------------------------
    def _check_config(self, levels, buckets, entries, count_levels):
        levels, buckets, count_levels = list(levels), list(buckets), list(count_levels)
        if levels or entries:
            if entries < 1 or entries > 8 or not buckets or len(buckets) > 127 or buckets[0] < 1 or any(
                    a >= b for a, b in zip(buckets, buckets[1:])):
                raise ValueError(f"need 1 <= entries <= 8 and buckets ascending from 1: {entries}, {buckets}")
            if any(k not in buckets for k in levels) or any(a >= b for a, b in zip(levels, levels[1:])):
                raise ValueError(f"levels must ascend and be of {buckets}: {levels}")
        if any(k < 1 for k in count_levels):
            raise ValueError(f"levels must be >= 1: {count_levels}")
        return tuple(levels), tuple(buckets), int(entries), tuple(count_levels)

    def prepare(self, levels, buckets, entries, count_levels) -> None:
        """Before the clock: advance()'s GPU state for this configuration, and per level the occurrences ordered by the
        step they become available in (online.rs :320-331)."""
        cfg = self._check_config(levels, buckets, entries, count_levels)
        if self.config is not None:
            if self.config != cfg:
                raise ValueError("advance()'s configuration is fixed by its first call")
            return
        self.config = cfg
        self.state = self._new_state(cfg)

    def _new_state(self, cfg, taus=None) -> dict:
        """advance()'s state; taus: (tau, tau_in) in place of the spans' (the rule "segment"'s)."""
        levels, buckets, entries, count_levels = cfg
        dev, n = self.dev, self.n
        tau_all, tau_in_all = taus if taus is not None else (self.tau, self.tau_in)
        E = max(1, entries)
        st = {"levels": {}, "E": E}
        # queries: positions trained as inputs, by step
        q_valid = tau_in_all != NONE
        q_pos = torch.nonzero(q_valid).squeeze(1)
        q_step = tau_in_all[q_pos]
        order = torch.sort(q_step, stable=True).indices
        st["q_pos"] = q_pos[order].to(torch.int32).contiguous()
        st["q_step"] = q_step[order].cpu().numpy()
        idx = torch.arange(n, device=dev)
        for k in sorted(set(levels) | set(count_levels)):
            # occurrences ending at g: tokens g-k+1..g and next g+1 within g's part; alpha = 1 + max tau over them
            ok = (idx - k + 1 >= self.part_lo) & (idx + 1 < self.part_hi)
            a = torch.full((n,), -1, dtype=torch.int64, device=dev)
            for d in range(-k + 1, 2):
                sh = torch.full((n,), NONE, dtype=torch.int64, device=dev)
                lo, hi = max(0, -d), min(n, n - d)
                if hi > lo:
                    sh[lo:hi] = tau_all[lo + d : hi + d]
                a = torch.maximum(a, sh)
            ok &= a != NONE
            occ = torch.nonzero(ok).squeeze(1)
            alpha = a[occ] + 1
            o = torch.sort(alpha, stable=True).indices
            m = int(occ.numel())
            cap = max(1 << 16, int(m / LOAD) + 1)
            # the pair table: 16-byte slots (key, count); a record per context: total, distinct count and, where the
            # level keeps hint rows, its top entries (REC_TOP u32 words: one 64-byte line), else REC_CNT words
            pt = torch.full((cap, 2), -1, dtype=torch.int64, device=dev)
            pt[:, 1] = 0
            rw = REC_TOP if k in levels else REC_CNT
            st["levels"][k] = {
                "occ": occ[o].to(torch.int32).contiguous(), "alpha": alpha[o].cpu().numpy(),
                "ck": torch.full((cap,), -1, dtype=torch.int64, device=dev), "ccap": cap,
                "pt": pt, "pcap": cap, "rec": torch.zeros(cap * rw, dtype=torch.int32, device=dev), "rw": rw,
                "flags": torch.zeros(2, dtype=torch.int32, device=dev),
                "ctx_bits": max(1, (cap - 1).bit_length()),
            }
        # a step's events of every level go through one merge (ng_online_merge, or the sorted one), each level's pair
        # keys tagged with its index above the widest level's pair-key bits (ng_online_insert's tag, the merge's desc)
        st["tshift"] = 16 + max(lv["ctx_bits"] for lv in st["levels"].values())
        st["tag_bits"] = max(1, (len(st["levels"]) - 1).bit_length())
        if st["tshift"] + st["tag_bits"] > 64:
            raise ValueError("the online tables are too large for one step's tagged pair keys")
        desc = []
        for k, lv in st["levels"].items():
            desc += [lv["pt"].data_ptr(), lv["pcap"], lv["rec"].data_ptr(), int(lv["rw"] == REC_TOP),
                     lv["flags"].data_ptr()]
        st["top_desc"] = torch.tensor(desc, dtype=torch.int64, device=dev)
        per_step = np.zeros(1, np.int64)
        for lv in st["levels"].values():
            if len(lv["alpha"]):
                c = np.bincount(lv["alpha"])
                if len(c) > len(per_step):
                    per_step = np.pad(per_step, (0, len(c) - len(per_step)))
                per_step[: len(c)] += c
        most = max(1, int(per_step.max()))
        st["ev"] = torch.empty(most, dtype=torch.int64, device=dev)
        st["merge_temp"] = None
        if self.merge == "buckets":
            size = ctypes.c_size_t(0)
            try:
                self.lib("ng_online_merge", None, ctypes.c_void_p(ctypes.addressof(size)), None, most, None,
                         i32(len(st["levels"])), i32(st["tshift"]), i32(E))
            except RuntimeError:  # -1: the step is too large for the packed words; the sorted merge runs instead
                size = None
            if size is not None:
                st["merge_size"] = size
                st["merge_temp"] = torch.empty(max(1, size.value), dtype=torch.uint8, device=dev)
        if st["merge_temp"] is None:  # the sorted merge's buffers
            st["ev_sorted"] = torch.empty(most, dtype=torch.int64, device=dev)
            st["uk"] = torch.empty(most, dtype=torch.int64, device=dev)
            st["agg"] = torch.empty(most, dtype=torch.int32, device=dev)
            st["nruns"] = torch.zeros(1, dtype=torch.int64, device=dev)
            st["score"] = torch.empty(most, dtype=torch.int64, device=dev)
        nq = int(np.bincount(st["q_step"]).max()) if len(st["q_step"]) else 1
        st["qslot"] = {k: torch.empty(max(1, nq), dtype=torch.int32, device=dev) for k in levels}
        st["hinted"] = torch.zeros(1, dtype=torch.int32, device=dev)
        st["done"] = 0
        if levels:  # ng_online_rows' per-level descriptors (deepest first): the same buffers every step
            desc = []
            for k in sorted(levels, reverse=True):
                lv = st["levels"][k]
                desc += [st["qslot"][k].data_ptr(), lv["rec"].data_ptr(), buckets.index(k)]
            st["rows_desc"] = torch.tensor(desc, dtype=torch.int64, device=dev)
        return st

    def _range(self, arr: np.ndarray, lo: int, hi: int) -> tuple[int, int]:
        return int(np.searchsorted(arr, lo, side="left")), int(np.searchsorted(arr, hi, side="left"))

    def _step(self, st: dict, s: int, outs: dict, queries: bool = True) -> None:
        """Step s: its newly available occurrences inserted at every level, then (queries) its queries answered."""
        lib = self.lib
        levels, buckets, entries, count_levels = outs["cfg"]
        E = st["E"]
        m = 0
        ins = []
        for t, (k, lv) in enumerate(st["levels"].items()):
            a, b = self._range(lv["alpha"], s, s + 1)
            if b == a:
                continue
            # the pair counts and the contexts' records are updated per distinct pair and per context by the step's
            # merge, not per occurrence: no global atomic per occurrence, no chains of same-address atomics on hot
            # contexts
            ins.append((_ptr(lv["occ"], a), b - a, k, _ptr(lv["ck"]), lv["ccap"], _ptr(lv["pt"]), lv["pcap"],
                        _ptr(st["ev"], m), _ptr(lv["flags"]), t << st["tshift"]))
            m += b - a
        for j in range(0, len(ins), MAX_LAUNCH_LEVELS):  # every level's inserts in one launch
            part = ins[j : j + MAX_LAUNCH_LEVELS]
            lib("ng_online_insert_levels", self.tok, i32(len(part)), _i64_array(part), i32(0))
        if m and st["merge_temp"] is not None:
            lib("ng_online_merge", st["merge_temp"], ctypes.c_void_p(ctypes.addressof(st["merge_size"])), st["ev"], m,
                st["top_desc"], i32(len(st["levels"])), i32(st["tshift"]), i32(E))
        elif m:
            lib.cub("sort_pairs", st["ev"], st["ev_sorted"], None, None, m, i32(0), i32(st["tshift"] + st["tag_bits"]))
            lib.cub("reduce_by_key", st["ev_sorted"], st["uk"], None, st["agg"], st["nruns"], m)  # run lengths
            lib("ng_online_top", st["uk"], st["nruns"], m, st["agg"], st["top_desc"], i32(len(st["levels"])),
                i32(st["tshift"]), st["score"], i32(E), i32(1))
        qa, qb = self._range(st["q_step"], s, s + 1)
        mq = qb - qa
        if mq == 0 or not queries:
            return
        qpos = st["q_pos"][qa:qb]
        qry = []
        nc = len(count_levels)
        for k in list(count_levels) + [k for k in levels if k not in count_levels]:
            lv = st["levels"][k]
            ci = count_levels.index(k) if k in count_levels else -1
            qry.append((k, _ptr(lv["ck"]), lv["ccap"], _ptr(lv["pt"]), lv["pcap"], _ptr(lv["rec"]), lv["rw"],
                        _ptr(st["qslot"][k]) if k in levels else 0,
                        _ptr(outs["tot"]) if ci >= 0 else 0, _ptr(outs["dist"]) if ci >= 0 else 0,
                        _ptr(outs["cnt"]) if ci >= 0 else 0, nc if ci >= 0 else 1, max(ci, 0)))
        for j in range(0, len(qry), MAX_LAUNCH_LEVELS):  # every level's queries in one launch
            part = qry[j : j + MAX_LAUNCH_LEVELS]
            lib("ng_online_query_levels", self.tok, self.avail, self.has_next, qpos, mq, i32(len(part)),
                _i64_array(part))
        if levels:
            lib("ng_online_rows", qpos, mq, i32(len(levels)), st["rows_desc"], i32(E), i32(outs["slots"]), outs["cell"],
                outs["next"], outs["weights"], outs["level"], st["hinted"])

    def _device_outputs(self, cfg, slots: int = 1, with_level: bool = False) -> dict:
        """Stream-sized outputs: hint rows in `slots` slots per position (cell [n, slots], next / weights [n, slots,
        entries], with_level the slots' bucket indices, -1 where empty) and count rows [n, len(count_levels)]."""
        levels, buckets, entries, count_levels = cfg
        n, dev = self.n, self.dev
        E = max(1, entries)
        return {"cfg": cfg, "slots": slots,
                "cell": torch.zeros((n, slots) if slots > 1 else n, dtype=torch.int16, device=dev),
                "next": torch.zeros((n, slots, E) if slots > 1 else (n, E), dtype=torch.int16, device=dev),
                "weights": torch.zeros((n, slots, E) if slots > 1 else (n, E), dtype=torch.int16, device=dev),
                "level": torch.full((n, slots), -1, dtype=torch.int8, device=dev) if with_level else None,
                "tot": torch.zeros((n, max(1, len(count_levels))), dtype=torch.int32, device=dev),
                "dist": torch.zeros((n, max(1, len(count_levels))), dtype=torch.int16, device=dev),
                "cnt": torch.zeros((n, max(1, len(count_levels))), dtype=torch.int32, device=dev)}

    def _check_flags(self, st) -> None:
        for k, lv in st["levels"].items():
            f = int(lv["flags"][0].item())
            if f & 4:
                raise RuntimeError(f"k={k}: a step's merge bucket needed more hash splits than the merge takes")
            if f:
                raise RuntimeError(f"k={k}: a table of the online state overflowed")

    @staticmethod
    def _copy_rows(outs: dict, rows: torch.Tensor, cell, nxt, weights, tot, dist, cnt) -> None:
        """The rows of `rows` (positions) from the device outputs into the caller's host arrays."""
        r = rows.long()
        rn = r.cpu().numpy()
        if cell is not None:
            cell[rn] = outs["cell"][r].cpu().numpy()
            nxt[rn] = outs["next"][r].cpu().numpy().view(np.uint16)
            weights[rn] = outs["weights"][r].cpu().numpy().view(np.uint16)
        if tot is not None:
            nc = tot.shape[1]
            tot[rn] = outs["tot"][r, :nc].cpu().numpy().view(np.uint32)
            dist[rn] = outs["dist"][r, :nc].cpu().numpy().view(np.uint16)
            cnt[rn] = outs["cnt"][r, :nc].cpu().numpy().view(np.uint32)

    def advance(self, step_hi: int, levels, buckets, entries: int, count_levels, cell=None, next=None, weights=None,
                tot=None, dist=None, cnt=None) -> int:
        """The rows of the queries trained in steps [done, step_hi) (what hints + counts write, rule "step"), with the
        counted occurrences kept between calls; returns the queries hinted (online.rs :333)."""
        self.prepare(levels, buckets, entries, count_levels)
        st = self.state
        if step_hi < self._done or step_hi >= 1 << 30:
            raise ValueError(f"bad step range [{self._done}, {step_hi})")
        if "outs" not in st:
            st["outs"] = self._device_outputs(self.config)
        outs = st["outs"]
        st["hinted"].zero_()
        for s in range(self._done, step_hi):
            self._step(st, s, outs)
        self._check_flags(st)
        qa, qb = self._range(st["q_step"], self._done, step_hi)
        if cell is not None or tot is not None:
            self._copy_rows(outs, st["q_pos"][qa:qb], cell, next, weights, tot, dist, cnt)
        self._done = step_hi
        return int(st["hinted"].item())

    def advance_device(self, step_hi: int) -> None:
        """advance() to step_hi with the prepared configuration, leaving the rows in GPU memory (self.state["outs"]),
        without synchronizing."""
        st = self.state
        if "outs" not in st:
            st["outs"] = self._device_outputs(self.config)
        outs = st["outs"]
        for s in range(self._done, step_hi):
            self._step(st, s, outs)
        self._done = step_hi

    def _range_rows(self, levels, buckets, entries, count_levels, step_lo, step_hi, rule, slots: int = 1,
                    with_level: bool = False):
        """A fresh state advanced over steps [0, step_hi), the queries of [step_lo, step_hi) answered. The rule
        "segment" (online.rs:14-17: every position a query at its segment's start, an occurrence counted iff its next
        token lies before that start) is the step rule with one step per segment in stream order: tau = tau_in = the
        position's segment index makes an occurrence's alpha 1 + the segment of its next token, so it counts for a
        query exactly when that segment lies before the query's; every step then runs as advance()'s do."""
        taus = None
        if rule == "segment":
            taus = (self.seg_index, self.seg_index)
            step_lo, step_hi = 0, int(self.seg_index[-1].item()) + 1
        elif rule != "step":
            raise ValueError(f"rule must be 'step' or 'segment': {rule}")
        if step_lo > step_hi or step_hi >= 1 << 30:
            raise ValueError(f"bad step range [{step_lo}, {step_hi})")
        cfg = self._check_config(levels, buckets, entries, count_levels)
        st = self._new_state(cfg, taus)
        outs = self._device_outputs(cfg, slots, with_level)
        for s in range(0, step_hi):  # earlier steps only insert their occurrences
            self._step(st, s, outs, queries=s >= step_lo)
        self._check_flags(st)
        qa, qb = self._range(st["q_step"], step_lo, step_hi)
        return st, outs, st["q_pos"][qa:qb]

    def segment_rows(self, levels, buckets, entries: int, slots: int = 1):
        """Every position's hint under the rule "segment" in `slots` slots, deepest levels first (train_hints.rs's
        rows of the stream: cell int16, next and weights uint16 [.., entries], level int8, -1 for an empty slot;
        [n] / [n, entries] with one slot, else [n, slots] / [n, slots, entries])."""
        st, outs, _ = self._range_rows(levels, buckets, entries, (), 0, 0, "segment", slots, True)
        lvl = outs["level"]
        return (outs["cell"].cpu().numpy(), outs["next"].cpu().numpy().view(np.uint16),
                outs["weights"].cpu().numpy().view(np.uint16), (lvl[:, 0] if slots == 1 else lvl).cpu().numpy())

    def segment_counts(self, levels):
        """Every position's count rows under the rule "segment" (train_counts.rs's): tot uint32, dist uint16, cnt
        uint32 [n, len(levels)]."""
        st, outs, _ = self._range_rows((), (1,), 0, levels, 0, 0, "segment")
        return (outs["tot"].cpu().numpy().view(np.uint32), outs["dist"].cpu().numpy().view(np.uint16),
                outs["cnt"].cpu().numpy().view(np.uint32))

    def hints(self, levels, buckets, entries, step_lo, step_hi, cell, next, weights, rule: str = "step") -> int:
        """The hint rows of the queries trained in steps [step_lo, step_hi), written into the stream-sized cell [n],
        next / weights [n, entries]; returns the queries hinted (online.rs :190)."""
        if entries < 1:
            raise ValueError("need entries >= 1")
        if len(cell) != self.n or next.shape != (self.n, entries) or weights.shape != (self.n, entries):
            raise ValueError(f"outputs must be [{self.n}] and [{self.n}, {entries}]")
        st, outs, rows = self._range_rows(levels, buckets, entries, (), step_lo, step_hi, rule)
        self._copy_rows(outs, rows, cell, next, weights, None, None, None)
        return int(st["hinted"].item())

    def counts(self, levels, step_lo, step_hi, tot, dist, cnt, rule: str = "step") -> None:
        """The count rows of the queries trained in steps [step_lo, step_hi) at each level, written into the
        stream-sized tot / dist / cnt [n, L] (online.rs :259)."""
        nl = len(levels)
        if not nl or min(levels) < 1:
            raise ValueError(f"levels must be >= 1: {levels}")
        if tot.shape != (self.n, nl) or dist.shape != (self.n, nl) or cnt.shape != (self.n, nl):
            raise ValueError(f"outputs must be [{self.n}, {nl}]")
        st, outs, rows = self._range_rows((), (1,), 0, levels, step_lo, step_hi, rule)
        self._copy_rows(outs, rows, None, None, None, tot, dist, cnt)
