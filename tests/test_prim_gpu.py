"""GPU: our device-wide primitives behind the CUB-style ABI calls (sort_pairs, inclusive_max, reduce_by_key) against
numpy (np.argsort kind="stable", np.maximum.accumulate, run sums) -- pinning the reference's CUB boundary -- and the
partition's first pass from segments (ng_seg_scatter: digit ranges, its capacity and region bounds)."""

import numpy as np
import pytest
import torch

from ngram_amd.lib import i32, u64

pytestmark = pytest.mark.gpu


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("n,b0,b1,dups", [(1, 0, 64, 0), (4095, 0, 64, 0), (4097, 0, 64, 16), (100_003, 16, 40, 1000),
                                           (300_000, 0, 64, 50), (70_000, 8, 8, 0), (65_536, 0, 12, 3),
                                           # 256 tiles (the scatter scans the digit counts itself), then 257 and more
                                           (2_097_152, 0, 64, 0), (2_097_153, 16, 48, 7), (5_000_000, 0, 40, 100)])
def test_sort_pairs_is_a_stable_radix_sort(lib, n, b0, b1, dups):
    rng = np.random.default_rng(n + b0)
    keys = rng.integers(0, 2 ** 63, size=n, dtype=np.int64).astype(np.uint64) * np.uint64(2) + \
        rng.integers(0, 2, size=n).astype(np.uint64)
    if dups:
        keys = rng.choice(keys[:dups], size=n)
    vals = np.arange(n, dtype=np.uint32)
    kin, vin = _t(keys.view(np.int64)), _t(vals.view(np.int32))
    kout, vout = torch.empty_like(kin), torch.empty_like(vin)
    lib.cub("sort_pairs", kin, kout, vin, vout, n, i32(b0), i32(b1))
    width = b1 - b0
    sk = (keys >> np.uint64(b0)) & np.uint64((1 << width) - 1) if width < 64 else keys
    order = np.argsort(sk, kind="stable")
    assert np.array_equal(vout.cpu().numpy().view(np.uint32), vals[order])
    assert np.array_equal(kout.cpu().numpy().view(np.uint64), keys[order])


@pytest.mark.parametrize("n,b0,b1", [(3_000_000, 0, 64), (20_000_000, 56, 64), (9_000_001, 20, 37)])
def test_sort_keys_only_across_many_tiles(lib, n, b0, b1):
    """Keys without values past 256 tiles (each pass's tile offsets from a histogram pass and a scan)."""
    rng = np.random.default_rng(n)
    keys = rng.integers(0, 2 ** 63, size=n, dtype=np.int64).astype(np.uint64) * np.uint64(2)
    kin = _t(keys.view(np.int64))
    kout = torch.empty_like(kin)
    lib.cub("sort_pairs", kin, kout, None, None, n, i32(b0), i32(b1))
    width = b1 - b0
    sk = (keys >> np.uint64(b0)) & np.uint64((1 << width) - 1) if width < 64 else keys
    assert np.array_equal(kout.cpu().numpy().view(np.uint64), keys[np.argsort(sk, kind="stable")])


def test_sort_pairs_empty_and_temp_query(lib):
    kin = torch.zeros(0, dtype=torch.int64, device="cuda")
    lib.cub("sort_pairs", kin, torch.empty_like(kin), None, None, 0, i32(0), i32(64))


@pytest.mark.parametrize("n", [1, 4096, 4097, 1_000_000, 17_000_000])
def test_inclusive_max(lib, n):
    rng = np.random.default_rng(n)
    a = rng.integers(-2 ** 40, 2 ** 40, size=n, dtype=np.int64)
    out = torch.empty(n, dtype=torch.int64, device="cuda")
    lib.cub("inclusive_max", _t(a), out, n)
    assert np.array_equal(out.cpu().numpy(), np.maximum.accumulate(a))


@pytest.mark.parametrize("n,runs", [(1, 1), (1000, 7), (100_000, 99_000), (2_000_000, 50), (3_000_000, 2_000_000)])
def test_reduce_by_key(lib, n, runs):
    rng = np.random.default_rng(n)
    keys = np.sort(rng.integers(0, runs, size=n)).astype(np.uint64) * np.uint64(977)
    vals = rng.integers(0, 2 ** 31, size=n, dtype=np.int64).astype(np.uint32)
    kout = torch.empty(n, dtype=torch.int64, device="cuda")
    vout = torch.empty(n, dtype=torch.int32, device="cuda")
    nr = torch.zeros(1, dtype=torch.int64, device="cuda")
    lib.cub("reduce_by_key", _t(keys.view(np.int64)), kout, _t(vals.view(np.int32)), vout, nr, n)
    u, first = np.unique(keys, return_index=True)
    sums = np.add.reduceat(vals.astype(np.uint64), first) & np.uint64(0xFFFFFFFF)
    m = int(nr.item())
    assert m == len(u)
    assert np.array_equal(kout[:m].cpu().numpy().view(np.uint64), u)
    assert np.array_equal(vout[:m].cpu().numpy().view(np.uint32), sums.astype(np.uint32))


@pytest.mark.parametrize("n,runs", [(1, 1), (1000, 7), (100_000, 99_000), (2_000_000, 50), (3_000_000, 2_000_000)])
def test_reduce_by_key_counting(lib, n, runs):
    """reduce_by_key without values: each item counts 1, so the outputs are the runs' lengths (np.unique's counts)."""
    rng = np.random.default_rng(n + 1)
    keys = np.sort(rng.integers(0, runs, size=n)).astype(np.uint64) * np.uint64(977)
    kout = torch.empty(n, dtype=torch.int64, device="cuda")
    vout = torch.empty(n, dtype=torch.int32, device="cuda")
    nr = torch.zeros(1, dtype=torch.int64, device="cuda")
    lib.cub("reduce_by_key", _t(keys.view(np.int64)), kout, None, vout, nr, n)
    u, counts = np.unique(keys, return_counts=True)
    m = int(nr.item())
    assert m == len(u)
    assert np.array_equal(kout[:m].cpu().numpy().view(np.uint64), u)
    assert np.array_equal(vout[:m].cpu().numpy(), counts.astype(np.int32))


@pytest.mark.parametrize("nbits", [8, 11])
def test_seg_scatter_groups_segments_by_digit(lib, nbits):
    """ng_seg_scatter from region segments: every key lands in its digit's range (the digit-major exclusive scan of the
    segments' digit histograms), each digit's keys the multiset numpy finds."""
    rng = np.random.default_rng(nbits)
    nseg, R = 37, 3000
    counts = rng.integers(0, R + 1, nseg).astype(np.uint32)
    counts[3] = 0
    shift = 64 - nbits
    keys = rng.integers(0, 1 << 63, (nseg, R), dtype=np.int64).astype(np.uint64) * np.uint64(2) + np.uint64(1)
    B = 1 << nbits
    digits = (keys >> np.uint64(shift)).astype(np.int64)
    hist = np.zeros((B, nseg), np.uint32)
    for s in range(nseg):
        np.add.at(hist[:, s], digits[s, : counts[s]], 1)
    dpre = (np.cumsum(hist.ravel()) - hist.ravel()).astype(np.uint32)
    n = int(counts.sum())
    out = torch.full((n + 64,), -1, dtype=torch.int64, device="cuda")
    regions = torch.from_numpy(keys.view(np.int64).ravel()).cuda()
    lib("ng_seg_scatter", regions, u64(R), None, torch.from_numpy(counts.view(np.int32)).cuda(),
        torch.from_numpy(dpre.view(np.int32)).cuda(), nseg, i32(shift), i32(nbits), out, u64(n))
    got = out.cpu().numpy().view(np.uint64)
    assert np.all(got[n:] == np.uint64(0xFFFFFFFFFFFFFFFF))  # nothing past n
    valid = np.concatenate([keys[s, : counts[s]] for s in range(nseg)])
    start = np.concatenate([np.zeros(1, np.int64), np.cumsum(hist.sum(1)).astype(np.int64)])
    for d in range(B):
        a, b = start[d], start[d + 1]
        assert np.array_equal(np.sort(got[a:b]), np.sort(valid[(valid >> np.uint64(shift)) == d]))


def test_seg_scatter_keeps_inside_its_capacity(lib):
    """A scatter launched before its host has checked the totals: histograms that promise more keys than the segments
    hold (an overflowed region), and a capacity below the total, write nothing past the capacity and read no region
    past R keys."""
    nseg, R, cap = 4, 256, 300
    keys = (np.arange(nseg * R, dtype=np.uint64) << np.uint64(2)) | np.uint64(1)
    counts = np.array([R + 500, 10, 0, 200], np.uint32)  # the first region claims more than it holds
    hist = np.zeros((256, nseg), np.uint32)
    hist[0, :] = [R + 500, 10, 0, 200]  # every key has digit 0 at shift 56 (the keys are small)
    dpre = (np.cumsum(hist.ravel()) - hist.ravel()).astype(np.uint32)
    guard = 4096
    out = torch.full((cap + guard,), -1, dtype=torch.int64, device="cuda")
    regions = torch.from_numpy(keys.view(np.int64)).cuda()
    lib("ng_seg_scatter", regions, u64(R), None, torch.from_numpy(counts.view(np.int32)).cuda(),
        torch.from_numpy(dpre.view(np.int32)).cuda(), nseg, i32(56), i32(8), out, u64(cap))
    got = out.cpu().numpy().view(np.uint64)
    assert np.all(got[cap:] == np.uint64(0xFFFFFFFFFFFFFFFF))
    # region 0 was read up to R keys: they fill places 0..R-1 (its digit range starts at 0)
    assert np.array_equal(np.sort(got[:R]), np.sort(keys[:R]))


@pytest.mark.parametrize("nwords", [0, 1, 255, 8191, 8192, 8193, 100_003])
@pytest.mark.parametrize("density", [0.0, 0.02, 0.5, 1.0])
@pytest.mark.parametrize("pre", [False, True])
def test_bits_list_matches_numpy(lib, nwords, density, pre):
    """ng_bits_list against numpy: every set bit's position in order and their count; with the prefix flag set, only
    the bits whose previous bit is set too (the bit before position 0 counts as set)."""
    rng = np.random.default_rng(nwords * 7 + int(density * 100) + pre)
    bits = rng.random(nwords * 32) < density
    words = np.packbits(bits.reshape(-1, 8)[:, ::-1], axis=1).reshape(-1).view("<u4") if nwords else np.zeros(0, "<u4")
    keep = bits.copy()
    if pre and nwords:
        keep &= np.concatenate([[True], bits[:-1]])
    want = np.flatnonzero(keep).astype(np.int64)
    bm = torch.from_numpy(words.view(np.int32).copy()).cuda()
    out = torch.full((max(len(want), 1),), -1, dtype=torch.int64, device="cuda")
    total = torch.zeros(1, dtype=torch.int64, device="cuda")
    flag = torch.tensor([1 if pre else 0], dtype=torch.int32, device="cuda")
    lib.cub("ng_bits_list", bm, nwords, out, total, flag)
    assert int(total.item()) == len(want)
    assert np.array_equal(out.cpu().numpy()[: len(want)], want)


@pytest.mark.parametrize("cap_frac", [1.0, 0.5, 0.0])
def test_bits_list32_keeps_the_first_cap(lib, cap_frac):
    """ng_bits_list32 (int32 positions, as the level pipeline lists the next level's query positions) against numpy:
    the first cap set bits' positions in order, nothing written past cap, and the count of every set bit."""
    rng = np.random.default_rng(int(cap_frac * 10))
    nwords = 70_001
    bits = rng.random(nwords * 32) < 0.3
    words = np.packbits(bits.reshape(-1, 8)[:, ::-1], axis=1).reshape(-1).view("<u4")
    want = np.flatnonzero(bits).astype(np.int64)
    cap = int(len(want) * cap_frac)
    bm = torch.from_numpy(words.view(np.int32).copy()).cuda()
    out = torch.full((cap + 64,), -7, dtype=torch.int32, device="cuda")
    total = torch.zeros(1, dtype=torch.int64, device="cuda")
    lib.cub("ng_bits_list32", bm, nwords, out, cap, total, None)
    o = out.cpu().numpy()
    assert int(total.item()) == len(want)
    assert np.array_equal(o[:cap], want[:cap])
    assert (o[cap:] == -7).all()


def test_pos_summary_hit_bits(lib):
    """ng_pos_summary's bitmap of the positions whose context occurred (dist > 0), the next level's list: bit i set
    exactly where ctx_of[i] >= 0 and dist[ctx_of[i]] > 0; zeros written for the others, over a ragged N."""
    rng = np.random.default_rng(5)
    N, n_ids = 100_003, 5000
    ctx_of = np.where(rng.random(N) < 0.8, rng.integers(0, n_ids, N), -1).astype(np.int32)
    dist = np.where(rng.random(n_ids) < 0.5, rng.integers(1, 9, n_ids), 0).astype(np.int32)
    rec = torch.zeros((n_ids, 4), dtype=torch.int32, device="cuda")
    outs = [torch.full((N,), -9, dtype=torch.int32, device="cuda") for _ in range(3)]
    tok = torch.full((N,), -9, dtype=torch.int16, device="cuda")
    tcnt = torch.full((N,), -9, dtype=torch.int32, device="cuda")
    hb = torch.full(((N + 63) // 64 * 2,), -1, dtype=torch.int32, device="cuda")
    lib("ng_pos_summary", torch.from_numpy(ctx_of).cuda(), N, 0, n_ids, None, rec, torch.from_numpy(dist).cuda(), None,
        None, i32(1), i32(1), i32(0), outs[0], outs[1], outs[2], tok, tcnt, None, hb)
    occ = (ctx_of >= 0) & (dist[np.maximum(ctx_of, 0)] > 0)
    got = np.unpackbits(hb.cpu().numpy().view(np.uint8), bitorder="little")[:N].astype(bool)
    assert np.array_equal(got, occ)
    assert np.array_equal(outs[1].cpu().numpy(), np.where(occ, dist[np.maximum(ctx_of, 0)], 0))
    assert (outs[2].cpu().numpy() == 0).all() and (tok.cpu().numpy()[~occ] == 0).all()
