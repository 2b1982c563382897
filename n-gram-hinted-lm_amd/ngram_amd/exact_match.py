"""exact_match's Python surface (exact_match/exact_match.pyi) on one MI355X: the query-filtered exact counts
`kgram_counts`, `kgram_query_counts` and `kgram_stats` (exact_match/src/kgram.rs :38-170), the corpus-wide
`CountTable` (count_table.py), the step-rule `OnlineRows` (online.py), and the module constants (lib.rs :25-32).
`train_hints` and `train_counts` (train_hints.rs, train_counts.rs: every training position's rows under the
segment rule) run on OnlineRows' rule "segment". The other CPU-only parts of the reference module (val_overlap,
val_scan, val_hint_rows, the approximate SlotIndex/StreamIndex) are not provided: looking them up raises
AttributeError.

Definitions (kgram.rs:7-9): a query position's k-context is its k tokens ending at it, valid iff they lie in its
segment (segments start at the first query token, at every BOS and, for kgram_query_counts, at each of `breaks`); an
occurrence is any k tokens within one shard followed by a token of the same shard. Context ids are this build's
(the distinct valid contexts in the order of their query-table slots, 0 .. C - 1); every output other than the ids
themselves is id-independent and equals the reference's. `memory` bounds the CPU build's working set and has no effect here;
`filter` (a bitmap of a smaller k) only saves probes there and is checked, not needed, here."""

from __future__ import annotations

import os

import numpy as np
import torch

from .count_table import CountTable  # noqa: F401  (part of the surface)
from .data import BOS, HEADER_BYTES, segments, shard_tokens
from .data import pack_layout as layout
from .lib import Lib, i32, u64
from .online import OnlineRows  # noqa: F401  (part of the surface)
from .qindex import QueryIndex

COUNTS = [2, 3, 5, 9, 17, 33]
PURITIES = [0.3, 0.5, 0.7, 0.85, 0.95]
LEVELS = [10, 20]
CELLS = (len(LEVELS) + 2) * (len(COUNTS) + 1) * (len(PURITIES) + 1)
LOAD = 0.7
NONE32 = 0xFFFFFFFF


def __getattr__(name: str):
    raise AttributeError(f"exact_match.{name} is not provided by the GPU build (CPU-only in the reference)")


def _validate(files, tokens, k, depth, memory) -> np.ndarray:
    t = np.ascontiguousarray(tokens, dtype=np.uint16)
    if not files or len(t) < 2 or k <= 0 or depth <= 0 or memory <= 0:
        raise ValueError("need files, 2+ tokens, and k, depth and memory > 0")
    if int(t.max()) > BOS:
        raise ValueError("invalid GPT-2 token")
    return t


def _corpus(files, train_tokens):
    """The shards (paths, or uint16 arrays), limited to their first train_tokens tokens, laid out on the GPU."""
    arrays = []
    left = None if train_tokens is None else int(train_tokens)
    for f in files:
        if isinstance(f, (str, bytes, os.PathLike)):
            n = shard_tokens(f)
            a = np.fromfile(f, dtype="<u2", count=n, offset=HEADER_BYTES)
        else:
            a = np.ascontiguousarray(f, dtype=np.uint16)
        if left is not None:
            a = a[:left]
            left -= len(a)
        arrays.append(a)
        if left is not None and left <= 0:
            break
    sizes = [len(a) for a in arrays]
    starts, L = layout(sizes)
    dev = torch.device("cuda", torch.cuda.current_device())
    tok = torch.full((L,), -1, dtype=torch.int16, device=dev)
    for a, st in zip(arrays, starts):
        if len(a):
            tok[st : st + len(a)].copy_(torch.from_numpy(a.view(np.int16)))
    return tok, sizes, starts, L


def _hits_bitmap(bm: torch.Tensor, sizes, starts) -> np.ndarray:
    """The scan's bitmap (one bit per position of the gapped layout) as the reference's: one bit per position of the
    shards concatenated, u64 words, bit p % 64 of word p // 64."""
    bits = np.unpackbits(bm.cpu().numpy().view(np.uint8), bitorder="little")
    flat = np.concatenate([bits[st : st + n] for st, n in zip(starts, sizes)]) if sizes else np.zeros(0, np.uint8)
    T = len(flat)
    pad = np.zeros((T + 63) // 64 * 64, np.uint8)
    pad[:T] = flat
    return np.packbits(pad, bitorder="little").view(np.uint64)


def _level(files, tokens: np.ndarray, k: int, top: int, train_tokens=None, breaks=(), cnt_top: int | None = None,
           depth: int = 0):
    lib = Lib()
    tok, sizes, starts, L = _corpus(files, train_tokens)
    dev = tok.device
    n = len(tokens) - 1
    x = torch.from_numpy(tokens[:-1].view(np.int16).copy()).to(dev)
    tgt = torch.from_numpy(tokens[1:].view(np.int16).copy()).to(dev)
    avail = torch.from_numpy(segments(tokens[:-1], list(breaks))).to(dev)
    vi = QueryIndex(lib, x, avail, k)
    grid = torch.cuda.get_device_properties(dev).multi_processor_count * 32
    T = sum(sizes)
    cap = max(1 << 16, int(min(T, 64 * vi.n + (1 << 20)) / LOAD))
    bm = torch.zeros(L // 32, dtype=torch.int32, device=dev)
    while True:
        keys = torch.full((cap,), -1, dtype=torch.int64, device=dev)
        cnts = torch.zeros(cap, dtype=torch.int32, device=dev)
        flags = torch.zeros(2, dtype=torch.int32, device=dev)
        lib("ng_scan_count", tok, L, i32(k), None, bm, vi.table, u64(vi.cap), vi.rep, x, keys, cnts, u64(cap), flags,
            i32(grid), i32(0))
        if int(flags[0].item()) == 0:
            break
        cap *= 2
    counter = torch.zeros(1, dtype=torch.int64, device=dev)
    ck = torch.empty(cap, dtype=torch.int64, device=dev)
    cc = torch.empty(cap, dtype=torch.int32, device=dev)
    lib("ng_table_compact", keys, cnts, u64(cap), ck, cc, counter)
    del keys, cnts
    U = int(counter.item())
    ids = vi.ids
    ctx_bits = max(1, (max(ids, 2) - 1).bit_length())
    uk = torch.empty(U, dtype=torch.int64, device=dev)
    agg = torch.empty(U, dtype=torch.int32, device=dev)
    if U:
        lib.cub("sort_pairs", ck, uk, cc, agg, U, i32(0), i32(16 + ctx_bits))
    del ck, cc
    start = torch.zeros(ids, dtype=torch.int64, device=dev)
    end = torch.zeros(ids, dtype=torch.int64, device=dev)
    lib("seg_bounds", uk, U, start, end)
    tot = torch.zeros(ids, dtype=torch.int64, device=dev)
    lib("ctx_tot", start, end, agg, ids, tot)
    # ranks: (context, count descending, token ascending), stable on the token order
    key2 = torch.empty(U, dtype=torch.int64, device=dev)
    val2 = torch.empty(U, dtype=torch.int32, device=dev)
    lib("rank_keys", uk, agg, U, key2, val2)
    k2s, sv = torch.empty_like(key2), torch.empty_like(val2)
    if U:
        lib.cub("sort_pairs", key2, k2s, val2, sv, U, i32(0), i32(32 + ctx_bits))
    del key2, k2s, val2
    rank_of = torch.empty(U, dtype=torch.int32, device=dev)
    lib("rank_scatter", sv, U, uk, agg, start, rank_of, None, None, i32(1))
    occupied = vi.table[:ids] != -1
    dense = torch.cumsum(occupied.to(torch.int64), 0) - 1
    C = int(occupied.sum().item())
    ctx = vi.ctx_of.long()
    key_of = torch.where(ctx >= 0, dense[ctx.clamp_min(0)], torch.full_like(ctx, NONE32))
    res = {"key_of": key_of.to(torch.int64).cpu().numpy().astype(np.uint32), "C": C}
    occ = occupied.nonzero().squeeze(1)
    dist_s = (end - start)
    res["totals"] = tot[occ].cpu().numpy().astype(np.uint64)
    res["distinct"] = dist_s[occ].cpu().numpy().astype(np.uint32)
    # the top `top` next tokens of each context in rank order, contexts in id order (= slot order)
    svl = sv.long()
    keep = rank_of[svl] < top
    ranked = svl[keep]
    res["next"] = (uk[ranked] & 0xFFFF).to(torch.int32).cpu().numpy().astype(np.uint16)
    res["next_counts"] = agg[ranked].cpu().numpy().view(np.uint32).copy()
    kept = torch.minimum(dist_s[occ], torch.full_like(dist_s[occ], top))
    res["offsets"] = np.concatenate([[0], np.cumsum(kept.cpu().numpy())]).astype(np.uint64)
    res["hits"] = _hits_bitmap(bm, sizes, starts)
    if cnt_top is not None:
        o = torch.zeros((3, n), dtype=torch.int32, device=dev)
        mask = torch.zeros(n, dtype=torch.int32, device=dev)
        lib("pos_outputs", vi.ctx_of, n, 0, ids, tgt, uk, agg, rank_of, start, end, tot, i32(0), i32(cnt_top),
            o[0], o[1], o[2], mask)
        res["cnt"] = o[2].cpu().numpy().view(np.uint32).copy()
    if depth:
        valid = ctx >= 0
        matched = valid & (tot[ctx.clamp_min(0)] > 0)
        want = (ctx.clamp_min(0) << 16) | (tgt.to(torch.int64) & 0xFFFF)
        j = torch.searchsorted(uk, want).clamp_max(max(U - 1, 0))
        found = matched & (uk[j] == want) if U else torch.zeros_like(matched)
        r = torch.where(found, rank_of[j].long(), torch.full_like(j, depth))
        r = r[found & (r < depth)]
        res["eligible"] = int(valid.sum().item())
        res["matched"] = int(matched.sum().item())
        res["ranks"] = torch.bincount(r, minlength=depth)[:depth].cpu().numpy().astype(np.uint64)
    return res


def _check_filter(files, train_tokens, filt) -> None:
    if filt is None:
        return
    T = 0
    for f in files:
        T += shard_tokens(f) if isinstance(f, (str, bytes, os.PathLike)) else len(f)
    if train_tokens is not None:
        T = min(T, int(train_tokens))
    if len(filt) != (T + 63) // 64:
        raise ValueError("filter is the bitmap of other files")


def kgram_counts(files, tokens, k: int, top: int, memory: int, train_tokens=None, filter=None):
    """Exact next-token counts of the query positions' k-contexts (kgram.rs :58-104): each position's context id
    (uint32, 2^32 - 1 where invalid); per context id its occurrences (uint64), distinct next tokens (uint32), offsets
    (uint64 [C + 1]) of its `top` most frequent next tokens (count descending, then token ascending) into next (uint16)
    and next_counts (uint32); the bitmap (uint64 words) of the corpus positions (the next tokens') whose k-context
    matched."""
    t = _validate(files, tokens, k, top, memory)
    _check_filter(files, train_tokens, filter)
    r = _level(files, t, k, top, train_tokens)
    return r["key_of"], r["totals"], r["distinct"], r["offsets"], r["next"], r["next_counts"], r["hits"]


def kgram_query_counts(files, tokens, k: int, top: int, cnt_top: int, memory: int, breaks=(), filter=None):
    """kgram_counts for a query of other shards concatenated (segments also start at each of `breaks`), then `cnt`:
    per query position the count of its next token among its context's cnt_top most frequent (kgram.rs :106-170)."""
    t = _validate(files, tokens, k, top, memory)
    if cnt_top <= 0 or any(b == 0 or b >= len(t) - 1 for b in breaks):
        raise ValueError("need cnt_top > 0 and breaks within the query")
    _check_filter(files, None, filter)
    r = _level(files, t, k, top, None, breaks, cnt_top)
    return (r["key_of"], r["totals"], r["distinct"], r["offsets"], r["next"], r["next_counts"], r["hits"], r["cnt"])


def kgram_stats(files, tokens, k: int, depth: int, memory: int, train_tokens=None, filter=None):
    """(eligible, matched, ranks, hits) of the query positions' k-contexts (kgram.rs :38-56, 237-278): positions with a
    valid k-context, those whose context occurred, per rank r < depth those whose next token is their context's
    (r + 1)-th most frequent (uint64 [depth]), and the corpus hit bitmap."""
    t = _validate(files, tokens, k, depth, memory)
    _check_filter(files, train_tokens, filter)
    r = _level(files, t, k, depth, train_tokens, depth=depth)
    return r["eligible"], r["matched"], r["ranks"], r["hits"]


TRAIN_BUCKETS = [2, 3, 4, 5, 6, 10, 20]  # train_hints.rs's default buckets (val_hints.py's LEVELS)


def _stream(files) -> tuple[np.ndarray, list[int]]:
    """The shards (paths, or uint16 arrays) in order as one host stream and its part bounds (empty shards hold no
    position and no part)."""
    arrays = []
    for f in files:
        if isinstance(f, (str, bytes, os.PathLike)):
            arrays.append(np.fromfile(f, dtype="<u2", count=shard_tokens(f), offset=HEADER_BYTES))
        else:
            arrays.append(np.ascontiguousarray(f, dtype=np.uint16))
    arrays = [a for a in arrays if len(a)]
    if not arrays:
        raise ValueError("the shards hold no tokens")
    bounds = np.concatenate([[0], np.cumsum([len(a) for a in arrays])]).astype(np.int64).tolist()
    return np.concatenate(arrays), bounds


def train_hints(files, levels, entries: int, buckets=None, slots: int = 1):
    """Every position of the shards `files` (in order): its hint over the variant `levels` in `slots` slots, the
    deepest levels whose context occurred before its segment, deepest first (train_hints.rs :41-110: a segment starts
    at each shard's first token and at every BOS; an occurrence, its k tokens and next token within one shard, counts
    iff its next token lies before the position's segment start). Returns cell int16, tokens and weights uint16
    [.., entries] and level int8 (the level's index in `buckets`, -1 for an empty slot): [N] and [N, entries] with one
    slot, else [N, slots] and [N, slots, entries]. Here at most 8 entries (the GPU's top lists)."""
    if not files or entries < 1 or not 1 <= slots <= 255:
        raise ValueError(f"need files, entries >= 1 and 1 <= slots <= 255: {len(files)} files, {entries} entries, "
                         f"{slots} slots")
    if entries > 8:
        raise ValueError(f"at most 8 entries on the GPU: {entries}")
    buckets = list(TRAIN_BUCKETS if buckets is None else buckets)
    levels = list(levels)
    if not buckets or len(buckets) > 127 or buckets[0] == 0 or any(a >= b for a, b in zip(buckets, buckets[1:])):
        raise ValueError(f"buckets must ascend from 1, at most 127 of them: {buckets}")
    if not levels or any(k not in buckets for k in levels) or any(a >= b for a, b in zip(levels, levels[1:])):
        raise ValueError(f"levels must ascend and be of {buckets}: {levels}")
    tokens, bounds = _stream(files)
    return OnlineRows(tokens, bounds, np.zeros((0, 3), np.int64)).segment_rows(levels, buckets, entries, slots)


def train_counts(files, levels):
    """Every position of the shards `files` (in order) and level k of `levels` (distinct, >= 1), over the occurrences
    of its k-context whose next token lies before its segment starts: tot uint32, dist uint16 and cnt uint32 [N, L]
    (train_counts.rs :20-48; cnt 0 for a shard's last position; all 0 where the k-context leaves the segment)."""
    levels = [int(k) for k in levels]
    if not files or not levels or min(levels) < 1 or len(set(levels)) != len(levels):
        raise ValueError(f"need files and distinct levels >= 1: {len(files)} files, levels {levels}")
    tokens, bounds = _stream(files)
    return OnlineRows(tokens, bounds, np.zeros((0, 3), np.int64)).segment_counts(levels)


def features(counts: torch.Tensor, nb: int = 25):
    """The count mixture's features (record_367_gpu_counts/track_1_short/counts/mix.py features :22-31) of
    counts int32 [3, L, n] on the GPU: tot, dist, min(cnt, tot) (float32 [n, L]), the bin parameter index
    clamp(floor(log2(max(tot, 1))), 0, nb - 1) + nb * level and the sparse-flag index (dist == 1) + 2 * level + nb * L
    (int64 [n, L]); one fused kernel (ng_features)."""
    if counts.dim() != 3 or counts.shape[0] != 3 or counts.dtype != torch.int32:
        raise ValueError("counts must be int32 [3, L, n]")
    counts = counts.contiguous()
    _, L, n = counts.shape
    dev = counts.device
    tot = torch.empty((n, L), dtype=torch.float32, device=dev)
    dist = torch.empty_like(tot)
    cnt = torch.empty_like(tot)
    b = torch.empty((n, L), dtype=torch.int64, device=dev)
    s = torch.empty_like(b)
    Lib()("ng_features", counts, i32(L), n, i32(nb), tot, dist, cnt, b, s)
    return tot, dist, cnt, b, s
