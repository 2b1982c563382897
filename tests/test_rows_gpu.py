"""GPU: the row kernels on hand-made inputs, against the oracle (itself pinned by hand in test_oracle.py): the record's
rows from per-context records (ng_record_rows: the 15-bit weight scaling above 32767, the depth choice, the clamped
top count), a batch of them (ng_batch_rows: padding, odd sizes, the overflow), and the count mixture's features at the
float32 edges of floor(log2) (ng_features)."""

import numpy as np
import pytest
import torch

import oracle as O
from ngram_amd.lib import Lib, i32

pytestmark = pytest.mark.gpu


def _records(tt: np.ndarray, tc: np.ndarray, tot: np.ndarray) -> torch.Tensor:
    """CtxRecord<8> words per context: total, pairs, 8 tokens two per word, 8 counts, the first word's index."""
    n = len(tot)
    r = np.zeros((n, 16), np.uint32)
    r[:, 0] = tot
    r[:, 1] = (tc > 0).sum(1)
    r[:, 2:6] = tt.astype(np.uint16).view(np.uint32).reshape(n, 4)
    r[:, 6:14] = tc
    return torch.from_numpy(r.view(np.int32)).cuda()


def _hand_case():
    tot = np.zeros((3, 4), np.uint32)
    tt = np.zeros((3, 4, 8), np.uint16)
    tc = np.zeros((3, 4, 8), np.uint32)
    tot[:, 0] = [4, 3, 0]
    tt[1, 0, :2], tc[1, 0, :2] = [7, 9], [2, 1]
    tt[0, 0, :1], tc[0, 0, :1] = [7], [4]
    tot[0, 1] = 40001
    tt[0, 1, :3], tc[0, 1, :3] = [5, 6, 8], [40000, 20000, 1]
    tot[:, 3] = 3_000_000_005
    tt[2, 3, :2], tc[2, 3, :2] = [11, 12], [3_000_000_000, 5]
    return tot, tt, tc


def test_record_rows_by_hand(gpu):
    tot, tt, tc = _hand_case()
    lib = Lib()
    n = tot.shape[1]
    ctx_of = torch.arange(n, dtype=torch.int32, device="cuda")  # position i's context is context i at every level
    rows = [torch.from_numpy(tot[r].view(np.int32)).cuda() for r in range(3)]
    recs = [_records(tt[r], tc[r], tot[r]) for r in range(3)]
    desc = torch.tensor([v for r in range(3) for v in (rows[r].data_ptr(), ctx_of.data_ptr(), recs[r].data_ptr())],
                        dtype=torch.int64, device="cuda")
    cells = torch.empty(n, dtype=torch.int32, device="cuda")
    entries = torch.empty((n, 8), dtype=torch.int32, device="cuda")
    lib("ng_record_rows", n, i32(3), desc, cells, entries)
    want_c, want_e = O.record_rows(tot, tt, tc)
    assert cells.cpu().tolist() == want_c.tolist() == [98, 83, 0, 165]
    assert np.array_equal(entries.cpu().numpy(), want_e)


@pytest.mark.parametrize("n,at,cap", [(3, 0, 5), (3, 1, 4), (4, 0, 9)])
def test_batch_rows_by_hand(gpu, n, at, cap):
    lib = Lib()
    cells = np.array([5, 0, 7, 9, 11], np.int32)
    entries = np.zeros((5, 8), np.int32)
    entries[0, :2] = [101, 102]
    entries[2, 0] = 103
    entries[3, 1] = 104
    entries[4, 7] = 105
    c = torch.from_numpy(cells).cuda()
    e = torch.from_numpy(entries).cuda()
    cc, ee = c[at : at + n].contiguous(), e[at : at + n].contiguous()
    out = torch.empty(n + 2 * cap, dtype=torch.int32, device="cuda")
    work = torch.empty(lib.size("ng_batch_rows_work", n), dtype=torch.int32, device="cuda")
    total = torch.zeros(1, dtype=torch.int64, device="cuda")
    lib("ng_batch_rows", cc, ee, n, cap, out, work, total)
    assert np.array_equal(out.cpu().numpy(), O.batch_rows(cells, entries, at, n, cap))
    assert int(total.item()) == int((entries[at : at + n] != 0).sum())


def test_batch_rows_many_tiles(gpu):
    """Past one tile of positions (the per-tile offsets' scan), an odd n, entries everywhere."""
    lib = Lib()
    rng = np.random.default_rng(4)
    n = 5001
    cells = rng.integers(0, 336, n).astype(np.int32)
    entries = np.where(rng.random((n, 8)) < 0.3, rng.integers(1, 1 << 30, (n, 8)), 0).astype(np.int32)
    cap = int((entries != 0).sum()) + 11
    out = torch.empty(n + 2 * cap, dtype=torch.int32, device="cuda")
    work = torch.empty(lib.size("ng_batch_rows_work", n), dtype=torch.int32, device="cuda")
    total = torch.zeros(1, dtype=torch.int64, device="cuda")
    lib("ng_batch_rows", torch.from_numpy(cells).cuda(), torch.from_numpy(entries).cuda(), n, cap, out, work, total)
    assert np.array_equal(out.cpu().numpy(), O.batch_rows(cells, entries, 0, n, cap))


def test_batch_rows_refuses_positions_past_its_offsets(gpu):
    """The tiles' offsets and the running offset are u32 (8 entries per position): n above (2^32 - 1) / 8 is refused
    before any launch (the buffers here are far smaller than such an n: nothing may be read)."""
    lib = Lib()
    small = torch.zeros(16, dtype=torch.int32, device="cuda")
    ent = torch.zeros((16, 8), dtype=torch.int32, device="cuda")
    total = torch.zeros(1, dtype=torch.int64, device="cuda")
    with pytest.raises(RuntimeError, match="returned -1"):
        lib("ng_batch_rows", small, ent, (0xFFFFFFFF // 8) + 1, 0, small, small, total)


def test_features_at_float32_edges(gpu):
    lib = Lib()
    ks = list(range(18, 26))
    tot = np.array([(1 << k) - 1 for k in ks] + [(1 << k) for k in ks] + [0, 1, 3], np.int64)
    n, L = len(tot), 1
    counts = np.zeros((3, L, n), np.int32)
    counts[0, 0] = tot.astype(np.uint32).view(np.int32)
    counts[1, 0] = np.arange(n) % 3
    counts[2, 0] = np.arange(n)
    dev = torch.from_numpy(counts).cuda()
    t, d, c = (torch.empty((n, L), dtype=torch.float32, device="cuda") for _ in range(3))
    b, s = (torch.empty((n, L), dtype=torch.int64, device="cuda") for _ in range(2))
    lib("ng_features", dev, i32(L), n, i32(25), t, d, c, b, s)
    want = O.features(counts)
    for got, w in zip((t, d, c, b, s), want):
        assert np.array_equal(got.cpu().numpy(), w)
