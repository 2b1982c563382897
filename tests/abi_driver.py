"""Test infrastructure: the reference-ABI libraries (libngram_amd.so's gpu_val_stats flavour, libngram_amd_record.so's
record flavour) driven through ctypes in the order a host that binds them calls them, so that their outputs can be
compared with the CPU oracle. The call order and buffer conventions are the ABI's (old_records/gpu_val_stats.py
ValIndex :604-651 and merge_level :988-1060, record_367_gpu_counts/track_1_short/counts/build.py :99-141, :205-371): the
query table of each level, the level's scan (counted, or emitted, grouped by sub-table and aggregated; a table that
overflows is doubled and the level scanned again), the pair table drained by owner, the owner's sort, segments,
totals, ranking and per-position outputs, then the variants' rows."""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ngram_amd.lib import i32, u64

EMPTY = -1  # u64 all-ones as int64


@dataclass
class QueryTable:
    table: torch.Tensor  # canonical linear-probing table (int64 keys, EMPTY-filled, ends with an empty slot)
    cap: int             # home slots umulhi(key, cap)
    rep: torch.Tensor    # int32 representative query position per slot
    ctx_of: torch.Tensor  # int32 context id (slot) per query position, -1 where invalid
    ids: int             # the id space (table slots)
    contexts: int


def query_table(lib, x, avail, k: int) -> QueryTable:
    """The distinct valid query k-contexts in canonical order (sorted keys, each at max(home, previous + 1))."""
    dev, n = x.device, x.numel()
    keys = torch.empty(n, dtype=torch.int64, device=dev)
    lib("val_keys", x, avail, n, i32(k), keys)
    pos = torch.nonzero(keys != EMPTY).squeeze(1)
    m = pos.numel()
    sk = torch.empty(max(m, 1), dtype=torch.int64, device=dev)
    sp = torch.empty(max(m, 1), dtype=torch.int32, device=dev)
    if m:
        lib.cub("sort_pairs", keys[pos].contiguous(), sk, pos.to(torch.int32), sp, m, i32(0), i32(64))
    sk, sp = sk[:m], sp[:m].long()
    first = torch.ones(m, dtype=torch.bool, device=dev)
    first[1:] = sk[1:] != sk[:-1]
    gid = torch.cumsum(first, 0) - 1
    uniq, reps = sk[first].contiguous(), sp[first].contiguous()
    C = uniq.numel()
    bad = torch.zeros(1, dtype=torch.int64, device=dev)
    lib("val_verify", x, sp, gid, reps, m, i32(k), bad)
    assert int(bad.item()) == 0, f"k={k}: query key collisions"
    cap = 2 * C + 64
    home = torch.empty(max(C, 1), dtype=torch.int64, device=dev)
    slot = torch.empty(max(C, 1), dtype=torch.int64, device=dev)
    if C:
        lib("val_homes", uniq, C, u64(cap), home)
        idx = torch.arange(C, device=dev)
        lib.cub("inclusive_max", (home[:C] - idx).contiguous(), slot, C)
        slot = slot[:C] + idx
    size = max(cap, int(slot[-1].item()) + 1 if C else 0) + 1
    table = torch.full((size,), EMPTY, dtype=torch.int64, device=dev)
    rep = torch.zeros(size, dtype=torch.int32, device=dev)
    ctx_of = torch.full((n,), -1, dtype=torch.int32, device=dev)
    if C:
        table[slot] = uniq
        rep[slot] = reps.to(torch.int32)
        ctx_of[sp] = slot[gid].to(torch.int32)
    return QueryTable(table, cap, rep, ctx_of, size, C)


def scan_and_count(lib, flavour: str, tok, L: int, k: int, bm_in, bm_out, qt: QueryTable, x, how: str, cap: int,
                   pbits: int = 2):
    """One level counted into a packed pair table: how = "count" (scan_level counting every position, or with bm_in
    the gated ones), "sparse" (gpu_val_stats mode 1 / record sparse), "emit" (mode 2 / record scan_emit), "words"
    (mode 3 / scan_emit words) -- the emitting ones then subpart_count, subpart_scatter and aggregate into 2^pbits
    sub-tables. Returns (pk, wraps, cap, reruns)."""
    dev = tok.device
    reruns = 0
    while True:
        flags = torch.zeros(2, dtype=torch.int32, device=dev)
        if how in ("count", "sparse"):
            pk = torch.full((cap,), EMPTY, dtype=torch.int64, device=dev)
            wraps = torch.zeros((cap + 3) // 4, dtype=torch.int32, device=dev)
            if flavour == "gvs":
                lib("scan_level", tok, L, i32(k), bm_in, bm_out, qt.table, u64(qt.cap), qt.rep, x, pk, wraps, u64(cap),
                    i32(0), flags, i32(0), i32(1 if how == "sparse" else 0), None, None)
            else:
                lib("scan_level", tok, L, i32(k), bm_in, bm_out, qt.table, u64(qt.cap), qt.rep, x, pk, wraps, u64(cap),
                    flags, i32(0), i32(how == "sparse"))
        else:
            emit = torch.empty(L, dtype=torch.int64, device=dev)
            emitted = torch.zeros(1, dtype=torch.int64, device=dev)
            if flavour == "gvs":
                lib("scan_level", tok, L, i32(k), bm_in, bm_out, qt.table, u64(qt.cap), qt.rep, x, None, None, u64(0),
                    i32(0), flags, i32(0), i32(3 if how == "words" else 2), emit, emitted)
            else:
                lib("scan_emit", tok, L, i32(k), bm_in, bm_out, qt.table, u64(qt.cap), qt.rep, x, flags, i32(0),
                    i32(how == "words"), emit, emitted)
            n = int(emitted.item())
            sub_cap = -(-cap // (1 << pbits))
            cap = sub_cap << pbits
            counts = torch.zeros(1 << pbits, dtype=torch.int64, device=dev)
            grouped = torch.empty(max(n, 1), dtype=torch.int64, device=dev)
            lib("subpart_count", emit, n, i32(pbits), counts)
            cursor = torch.cumsum(counts, 0) - counts
            lib("subpart_scatter", emit, n, i32(pbits), cursor, grouped)
            assert torch.equal(cursor, torch.cumsum(counts, 0)), "subpart_scatter filled every group"
            pk = torch.full((cap,), EMPTY, dtype=torch.int64, device=dev)
            wraps = torch.zeros((cap + 3) // 4, dtype=torch.int32, device=dev)
            lib("aggregate", grouped, n, pk, wraps, u64(sub_cap), i32(pbits), flags, i32(0))
        if int(flags[0].item()) == 0:
            return pk, wraps, cap, reruns
        reruns += 1
        cap *= 2


def drain(lib, pk, wraps, cap: int, bounds: list[int]):
    """The pair table's (key, count) entries grouped by owner (part_count + part_scatter): (keys, counts, per-owner
    counts)."""
    dev = pk.device
    W = len(bounds) - 1
    b = torch.tensor(bounds, dtype=torch.int64, device=dev)
    per = torch.zeros(W, dtype=torch.int64, device=dev)
    lib("part_count", pk, u64(cap), b, i32(W), per)
    U = int(per.sum().item())
    cursor = torch.cumsum(per, 0) - per
    keys = torch.empty(max(U, 1), dtype=torch.int64, device=dev)
    vals = torch.empty(max(U, 1), dtype=torch.int32, device=dev)
    lib("part_scatter", pk, wraps, u64(cap), b, i32(W), cursor, keys, vals)
    assert torch.equal(cursor, torch.cumsum(per, 0)), "part_scatter filled every owner's run"
    return keys[:U], vals[:U], per


def owner_outputs(lib, flavour: str, keys, vals, qt: QueryTable, tgt, li: int, out, mask, top: int, cnt_top: int):
    """Sort, segments, totals, ranks, tops and per-position outputs of one level: (top_tok, top_cnt, tot)."""
    dev = keys.device
    U, ids, N = keys.numel(), qt.ids, qt.ctx_of.numel()
    bits = max(1, (max(ids, 2) - 1).bit_length())
    uk = torch.empty(max(U, 1), dtype=torch.int64, device=dev)
    agg = torch.empty(max(U, 1), dtype=torch.int32, device=dev)
    if U:
        lib.cub("sort_pairs", keys, uk, vals, agg, U, i32(0), i32(16 + bits))
    start = torch.zeros(ids, dtype=torch.int64, device=dev)
    end = torch.zeros(ids, dtype=torch.int64, device=dev)
    lib("seg_bounds", uk, U, start, end)
    tot = torch.empty(ids, dtype=torch.int64, device=dev)
    lib("ctx_tot", start, end, agg, ids, tot)
    key2 = torch.empty(max(U, 1), dtype=torch.int64, device=dev)
    val2 = torch.empty(max(U, 1), dtype=torch.int32, device=dev)
    k2s, sv = torch.empty_like(key2), torch.empty_like(val2)
    lib("rank_keys", uk, agg, U, key2, val2)
    if U:
        lib.cub("sort_pairs", key2, k2s, val2, sv, U, i32(0), i32(32 + bits))
    top_tok = torch.zeros(ids * top, dtype=torch.int16, device=dev)
    top_cnt = torch.zeros(ids * top, dtype=torch.int32, device=dev)
    if flavour == "gvs":
        rank_of = torch.empty(max(U, 1), dtype=torch.int32, device=dev)
        lib("rank_scatter", sv, U, uk, agg, start, rank_of, top_tok, top_cnt, i32(top))
        lib("pos_outputs", qt.ctx_of, N, 0, ids, tgt, uk, agg, rank_of, start, end, tot, i32(li), i32(cnt_top),
            out[0, li], out[1, li], out[2, li], mask)
    else:
        lib("rank_scatter", sv, U, uk, agg, start, top_tok, top_cnt, i32(top))
        lib("pos_outputs", qt.ctx_of, N, 0, ids, tgt, uk, agg, start, end, tot, out[0, li], out[1, li], out[2, li])
    return top_tok, top_cnt, tot


def level_stats(lib, flavour: str, tok, L: int, x, tgt, avail, levels, how: str = "count", cap: int = 1 << 16,
                top: int = 8, cnt_top: int = 1024):
    """Every level in turn (each gated by the previous level's hit bitmap): counts int32 [3, len(levels), N], the
    mask, and per level (query table, top_tok, top_cnt, tot, reruns)."""
    dev, N = tok.device, x.numel()
    out = torch.zeros((3, len(levels), N), dtype=torch.int32, device=dev)
    mask = torch.zeros(N, dtype=torch.int32, device=dev)
    bm_prev, per = None, {}
    for li, k in enumerate(levels):
        qt = query_table(lib, x, avail, k)
        bm = torch.zeros(L // 32, dtype=torch.int32, device=dev)
        mode = how if bm_prev is not None or how in ("count", "emit") else {"sparse": "count", "words": "emit"}[how]
        pk, wraps, c, reruns = scan_and_count(lib, flavour, tok, L, k, bm_prev, bm, qt, x, mode, cap)
        keys, vals, _ = drain(lib, pk, wraps, c, [0, qt.ids])
        del pk, wraps
        tops = owner_outputs(lib, flavour, keys, vals, qt, tgt, li, out, mask, top, cnt_top)
        per[k] = (qt, *tops, reruns)
        bm_prev = bm
    return out, mask, per


def variant_rows(lib, N: int, mask, per: dict, levels, variant, buckets):
    """One variant's rows (int32 [N, 9]) from level_stats' tops."""
    dev = mask.device
    desc = []
    for k in variant:
        qt, top_tok, top_cnt, tot, _ = per[k]
        desc += [levels.index(k), buckets.index(k), qt.ctx_of.data_ptr(), 0, qt.ids, top_tok.data_ptr(),
                 top_cnt.data_ptr(), tot.data_ptr()]
    d = torch.tensor(desc, dtype=torch.int64, device=dev)
    rows = torch.zeros((N, 9), dtype=torch.int32, device=dev)
    lib("variant_rows", N, mask, i32(len(variant)), d, rows)
    torch.cuda.synchronize()  # the descriptor's pointers are read by the kernel
    return rows
