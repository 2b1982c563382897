"""GPU: the 32-bit count's passes (pairs32.hip) on their own against numpy: the second, most-significant-digit-first
pass (ng_msd_pass: every bucket's keys sub-grouped by the next digit, the partitions' starts) and the first pass's
narrowing scatter (ng_seg_scatter_narrow), with empty buckets, a bucket spanning many tiles, and keys placed beyond
the capacity dropped; the count's runs mode with the records made from its runs (ng_part_count32, ng_ctx_agg_runs)."""

import numpy as np
import pytest
import torch

from ngram_amd.lib import i32, u64

pytestmark = pytest.mark.gpu


def _msd(lib, sizes, nb_bits, nbits, shift, seed=0):
    rng = np.random.default_rng(seed)
    nb = 1 << nb_bits
    assert len(sizes) == nb
    total = int(sum(sizes))
    keys = rng.integers(0, 1 << 32, total, dtype=np.uint64).astype(np.uint32)
    starts = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    # dpre as a first pass leaves it for one segment: digit b's offset
    nseg = 1
    dpre = torch.from_numpy(starts[:-1].astype(np.uint32).view(np.int32)).cuda()
    tot = torch.tensor([total], dtype=torch.int64, device="cuda")
    cap = total + 100
    kin = torch.zeros(cap, dtype=torch.int32, device="cuda")
    kin[:total] = torch.from_numpy(keys.view(np.int32)).cuda()
    out = torch.full((cap,), -1, dtype=torch.int32, device="cuda")
    P = nb << nbits
    start = torch.empty(P + 1, dtype=torch.int64, device="cuda")
    lib.cub("ng_msd_pass", kin, dpre, nseg, i32(nb_bits), tot, u64(cap), i32(shift), i32(nbits), out, start)
    o = out.cpu().numpy().view(np.uint32)[:total]
    st = start.cpu().numpy()
    assert st[0] == 0 and st[-1] == total and (np.diff(st) >= 0).all()
    for b in range(nb):
        kb = keys[starts[b] : starts[b + 1]]
        dig = (kb >> shift) & ((1 << nbits) - 1)
        for d in np.unique(dig) if len(kb) else []:
            p = (b << nbits) | int(d)
            got = np.sort(o[st[p] : st[p + 1]])
            assert np.array_equal(got, np.sort(kb[dig == d])), (b, d)
        # partitions of digits absent from the bucket are empty
        present = set(np.unique(dig).tolist()) if len(kb) else set()
        for d in range(1 << nbits):
            if d not in present:
                p = (b << nbits) | d
                assert st[p] == st[p + 1], (b, d)
    assert (out.cpu().numpy()[total:] == -1).all()


def test_msd_pass_small(lib):
    sizes = [0, 5, 1, 0, 100, 0, 0, 3] + [7] * 248
    _msd(lib, sizes, 8, 3, 5)


def test_msd_pass_bucket_of_many_tiles(lib):
    sizes = [0] * 256
    sizes[3] = 200_000  # 13 tiles of 16384 keys
    sizes[200] = 16_384
    sizes[255] = 16_385
    _msd(lib, sizes, 8, 11, 21, seed=1)


def test_msd_pass_wide_buckets(lib):
    rng = np.random.default_rng(2)
    sizes = rng.integers(0, 3000, 1024).tolist()
    _msd(lib, sizes, 10, 7, 25, seed=3)


def test_seg_scatter_narrow(lib):
    """Region segments of u64 keys scattered by their digit at bit 28 (4 bits) and narrowed to the low 32 bits."""
    rng = np.random.default_rng(4)
    nseg, R = 5, 3000
    counts = rng.integers(0, R + 1, nseg).astype(np.uint32)
    counts[2] = 0
    regions = rng.integers(0, 1 << 32, nseg * R, dtype=np.uint64)  # keys below 2^32: digit bits [28, 32)
    shift, nbits = 28, 4
    hist = np.zeros((1 << nbits, nseg), np.uint32)
    for s in range(nseg):
        k = regions[s * R : s * R + counts[s]]
        hist[:, s] = np.bincount((k >> shift) & 15, minlength=16)
    flat = hist.reshape(-1)
    dpre = np.concatenate([[0], np.cumsum(flat)[:-1]]).astype(np.uint32)
    total = int(flat.sum())
    out = torch.full((total,), -1, dtype=torch.int32, device="cuda")
    lib("ng_seg_scatter_narrow", torch.from_numpy(regions.view(np.int64)).cuda(), u64(R), None,
        torch.from_numpy(counts.view(np.int32)).cuda(), torch.from_numpy(dpre.view(np.int32)).cuda(), nseg,
        i32(shift), i32(nbits), out, u64(total))
    o = out.cpu().numpy().view(np.uint32)
    allk = np.concatenate([regions[s * R : s * R + counts[s]] for s in range(nseg)]).astype(np.uint32)
    starts = np.concatenate([[0], np.cumsum(hist.sum(axis=1))]).astype(np.int64)
    for d in range(16):
        seg = o[starts[d] : starts[d + 1]]
        assert np.array_equal(np.sort(seg), np.sort(allk[((allk >> shift) & 15) == d])), d


def test_msd_pass64_words_by_context(lib):
    """The words' second pass: u64 keys grouped by their top 11 bits, sub-grouped by the next 4 (ng_msd_pass64), and
    the buckets' starts alone (nbits 0)."""
    rng = np.random.default_rng(5)
    n = 300_000
    keys = rng.integers(0, 1 << 63, n, dtype=np.uint64) * np.uint64(2) + rng.integers(0, 2, n, dtype=np.uint64)
    top = (keys >> np.uint64(53)).astype(np.int64)
    order = np.argsort(top, kind="stable")
    keys = keys[order]
    counts = np.bincount(top, minlength=2048)
    starts = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    dpre = torch.from_numpy(starts[:-1].astype(np.uint32).view(np.int32)).cuda()
    tot = torch.tensor([n], dtype=torch.int64, device="cuda")
    kin = torch.from_numpy(keys.view(np.int64)).cuda()
    out = torch.empty(n, dtype=torch.int64, device="cuda")
    start = torch.empty(2048 * 16 + 1, dtype=torch.int64, device="cuda")
    lib.cub("ng_msd_pass64", kin, dpre, 1, i32(11), tot, u64(n), i32(49), i32(4), out, start)
    o = out.cpu().numpy().view(np.uint64)
    st = start.cpu().numpy()
    sub = (keys >> np.uint64(49)).astype(np.int64)  # bucket << 4 | digit
    cnt = np.bincount(sub, minlength=2048 * 16)
    assert np.array_equal(st, np.concatenate([[0], np.cumsum(cnt)]))
    for p in np.unique(sub)[:: 97]:
        assert np.array_equal(np.sort(o[st[p] : st[p + 1]]), np.sort(keys[sub == p])), p
    bst = torch.empty(2049, dtype=torch.int64, device="cuda")
    lib.cub("ng_msd_pass64", None, dpre, 1, i32(11), tot, u64(n), i32(0), i32(0), None, bst)
    assert np.array_equal(bst.cpu().numpy(), starts)


@pytest.mark.parametrize("cap_frac", [1.0, 0.5])
def test_select_positive(lib, cap_frac):
    """ng_select_positive: the positive entries' positions in order and their count, the count exact even when the
    list is cut at cap."""
    rng = np.random.default_rng(6)
    n = 1_000_003
    v = rng.integers(-3, 3, n).astype(np.int32)
    want = np.nonzero(v > 0)[0]
    cap = int(len(want) * cap_frac)
    out = torch.full((max(cap, 1),), -7, dtype=torch.int32, device="cuda")
    nd = torch.empty(1, dtype=torch.int64, device="cuda")
    lib.cub("ng_select_positive", torch.from_numpy(v).cuda(), n, out, cap, nd)
    assert int(nd.item()) == len(want)
    assert np.array_equal(out.cpu().numpy()[:cap], want[:cap])


def _wmix(x, W):
    """part.h's wmix: a bijection of W-bit values (two odd multiplications, two xor-shifts by ceil(W / 2))."""
    m, s = np.uint64((1 << W) - 1), np.uint64((W + 1) >> 1)
    x = (x * np.uint64(0x9E3779B97F4A7C15)) & m
    x ^= x >> s
    x = (x * np.uint64(0xBF58476D1CE4E5B9)) & m
    return x ^ (x >> s)


def _kmix(x, W, M):
    lo = np.uint64((1 << M) - 1)
    return (x & ~lo & np.uint64((1 << W) - 1)) | _wmix(x & lo, M)


@pytest.mark.parametrize("n_ids,n_ev,d2,kt", [(5000, 60_000, 3, 4), (3_000_000, 4_000_000, 8, 4),
                                              (3_000_000, 2_000_000, 6, 8), (700_000, 1_500_000, 2, 1)])
def test_count32_runs_records(lib, n_ids, n_ev, d2, kt):
    """The count's runs mode and the records made from its runs (ng_part_count32 with runs, ng_ctx_agg_runs) against
    numpy: events keyed by context range (kmix with M = W - d1), partitioned by their top d1 + d2 bits; every id's pair
    count and every present context's record (total, pairs, top kt by count then token). n_ids below a power of two
    leaves the trailing partitions empty (the last block's fast exit); (5000, d2 3) has one group per bucket, (3M,
    d2 8) 256 runs a group and 8 groups a bucket."""
    from ngram_amd import partcount as P

    rng = np.random.default_rng(n_ids + d2)
    idb, W = P.w_bits(n_ids)
    d1 = P.first_digit(W)
    M = W - d1
    pbits = d1 + d2
    agg = P.AGG_ID_BITS - 1 if kt >= 8 else P.AGG_ID_BITS
    ibits = min(agg, idb - d1)
    gbits = idb - d1 - ibits
    assert gbits <= 6
    hot = rng.integers(0, n_ids, 50)
    ids = np.where(rng.random(n_ev) < 0.2, hot[rng.integers(0, 50, n_ev)], rng.integers(0, n_ids, n_ev))
    toks = (rng.zipf(1.3, n_ev) - 1) % 65536
    pk = (ids.astype(np.uint64) << np.uint64(16)) | toks.astype(np.uint64)
    ek = _kmix(pk, W, M)
    part = (ek >> np.uint64(W - pbits)).astype(np.int64)
    order = np.argsort(part, kind="stable")
    P_ = 1 << pbits
    start = np.searchsorted(part[order], np.arange(P_ + 1)).astype(np.int64)
    ev = (ek[order] & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    cb = idb
    G = 256
    dev = "cuda"
    ev_d = torch.from_numpy(ev.view(np.int32)).to(dev)
    start_d = torch.from_numpy(start).to(dev)
    qstart = torch.zeros(P_ + 1, dtype=torch.int64, device=dev)
    out_k = torch.empty(n_ev, dtype=torch.int64, device=dev)
    esc_k = torch.full((P.ESC_CAP,), -1, dtype=torch.int64, device=dev)
    esc_c = torch.empty(P.ESC_CAP, dtype=torch.int32, device=dev)
    seg_cnt = torch.empty(G, dtype=torch.int32, device=dev)
    seg_base = torch.empty(G, dtype=torch.int64, device=dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    runs = torch.empty(P_ << gbits, dtype=torch.int64, device=dev)
    live_np = (((n_ids - 1) >> (idb - d1)) + 1) << d2
    n_words = torch.zeros(1, dtype=torch.int64, device=dev)
    lib("ng_part_count32", ev_d, start_d, i32(pbits), i32(W), i32(M), None, None, qstart, out_k, i32(cb), esc_k, esc_c,
        u64(P.ESC_CAP), seg_cnt, seg_base, None, None, i32(0), i32(0), __import__("ctypes").c_uint32(P.P32_LIMIT), flags,
        i32(G), None, runs, i32(gbits), i32(16 + ibits), i32(d2), live_np, n_words)
    rec = torch.zeros((n_ids, P.RECORD_WORDS[kt]), dtype=torch.int32, device=dev)
    dist = torch.empty(n_ids, dtype=torch.int32, device=dev)
    lib("ng_ctx_agg_runs", out_k, runs, 1 << (d1 + gbits), i32(d2), i32(gbits), i32(ibits), i32(cb), n_ids, esc_k,
        esc_c, u64(P.ESC_CAP), i32(kt), rec, dist, flags, None, i32(0))
    assert int(flags.item()) == 0
    # numpy: distinct pairs with counts, per context
    up, cnt = np.unique(pk, return_counts=True)
    assert int(n_words.item()) == len(up)
    c_of = (up >> np.uint64(16)).astype(np.int64)
    t_of = (up & np.uint64(0xFFFF)).astype(np.int64)
    want_dist = np.bincount(c_of, minlength=n_ids)
    assert np.array_equal(dist.cpu().numpy(), want_dist)
    want_tot = np.bincount(c_of, weights=cnt, minlength=n_ids).astype(np.int64)
    r = rec.cpu().numpy().view(np.uint32)
    present = np.nonzero(want_dist)[0]
    assert np.array_equal(r[present, 0].astype(np.int64), want_tot[present])
    assert np.array_equal(r[present, 1].astype(np.int64), want_dist[present])
    # top kt: count descending, then token ascending
    o = np.lexsort((t_of, -cnt, c_of))
    c_s, t_s, n_s = c_of[o], t_of[o], cnt[o]
    first = np.searchsorted(c_s, present)
    tokw = (kt + 1) // 2
    for rr in range(kt):
        idx = first + rr
        ok = (idx < len(c_s)) & (c_s[np.minimum(idx, len(c_s) - 1)] == present)
        tok_w = (r[present, 2 + rr // 2] >> (16 * (rr & 1))) & 0xFFFF
        cnt_w = r[present, 2 + tokw + rr]
        want_t = np.where(ok, t_s[np.minimum(idx, len(c_s) - 1)], 0)
        want_n = np.where(ok, n_s[np.minimum(idx, len(c_s) - 1)], 0)
        assert np.array_equal(tok_w.astype(np.int64), want_t), rr
        assert np.array_equal(cnt_w.astype(np.int64), want_n), rr
