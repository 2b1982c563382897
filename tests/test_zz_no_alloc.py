"""GPU: ng_batch_rows_noalloc (the batch rows without a workspace argument: its per-tile offsets in the library's own
device array) through the C ABI against ng_batch_rows with an allocated workspace: two calls in a row, the second
smaller (the array keeps the first call's contents), and a size past the array refused before any launch."""

import numpy as np
import pytest
import torch

from ngram_amd.lib import Lib

pytestmark = pytest.mark.gpu

MAX_POSITIONS = 65536 * 1024  # the entry point's limit (its array holds 65536 tiles of 1024 positions)


def _inputs(rng, n):
    cells = torch.from_numpy(rng.integers(0, 336, n).astype(np.int32)).cuda()
    e = np.where(rng.random((n, 8)) < 0.25, rng.integers(1, 1 << 30, (n, 8)), 0).astype(np.int32)
    return cells, torch.from_numpy(e).cuda(), int((e != 0).sum())


def test_no_alloc_batch_rows_matches_the_workspace_version(gpu):
    lib = Lib()
    rng = np.random.default_rng(12)
    for n in (300_001, 5_003):  # the second call smaller: the array still holds the first call's offsets
        cells, entries, m = _inputs(rng, n)
        cap = m + 17
        want = torch.empty(n + 2 * cap, dtype=torch.int32, device="cuda")
        work = torch.empty(lib.size("ng_batch_rows_work", n), dtype=torch.int32, device="cuda")
        t_want = torch.zeros(1, dtype=torch.int64, device="cuda")
        lib("ng_batch_rows", cells, entries, n, cap, want, work, t_want)
        got = torch.full((n + 2 * cap,), -7, dtype=torch.int32, device="cuda")
        t_got = torch.full((1,), -7, dtype=torch.int64, device="cuda")
        lib("ng_batch_rows_noalloc", cells, entries, n, cap, got, t_got)
        assert torch.equal(got, want) and int(t_got.item()) == int(t_want.item()) == m
    # the capacity exceeded: the same total, only capacity pairs written (the caller raises)
    cells, entries, m = _inputs(rng, 4000)
    got = torch.zeros(4000 + 2 * 10, dtype=torch.int32, device="cuda")
    t_got = torch.zeros(1, dtype=torch.int64, device="cuda")
    lib("ng_batch_rows_noalloc", cells, entries, 4000, 10, got, t_got)
    assert int(t_got.item()) == m > 10


def test_no_alloc_batch_rows_refuses_more_than_its_array(gpu):
    lib = Lib()
    cells = torch.zeros(8, dtype=torch.int32, device="cuda")
    entries = torch.zeros((8, 8), dtype=torch.int32, device="cuda")
    out = torch.zeros(8, dtype=torch.int32, device="cuda")
    total = torch.zeros(1, dtype=torch.int64, device="cuda")
    with pytest.raises(RuntimeError, match="returned -1"):  # refused on the host, before any launch
        lib("ng_batch_rows_noalloc", cells, entries, MAX_POSITIONS + 1, 0, out, total)
