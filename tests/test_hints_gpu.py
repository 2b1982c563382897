"""GPU: the hint directory's reader on the device (ng_hint_widen, ng_count_rows through the staged ring) against the
same reader on the CPU and against torch's own widening on the GPU (the reference's expressions), and a directory
written from the validation statistics' outputs read back position by position."""

import numpy as np
import pytest
import torch

from ngram_amd import data
from ngram_amd import gpu_val_stats as G
from ngram_amd import hints as H

pytestmark = pytest.mark.gpu


def _rows(rng, n, slots=1):
    lead = (n,) if slots == 1 else (n, slots)
    hinted = rng.random(lead) < 0.6
    cell = np.where(hinted, rng.integers(1, 336, lead), 0).astype(np.int16)
    counts = np.sort(rng.integers(0, 1 << 16, (*lead, 8)), -1)[..., ::-1] * hinted[..., None]
    return cell, rng.integers(0, 65536, (*lead, 8)).astype(np.uint16), H.weights(counts)


@pytest.fixture(scope="module")
def hint_dir(tmp_path_factory):
    rng = np.random.default_rng(5)
    L = len(H.FAKE_COUNT_LEVELS)
    tot = rng.integers(0, 1 << 32, (20_000, L), dtype=np.uint64).astype(np.uint32)  # above 2^24: rounded to float32
    counts = (tot, np.minimum(tot, rng.integers(0, 65536, (20_000, L))).astype(np.uint16),
              (rng.random((20_000, L)) * tot).astype(np.uint32))
    d = H.write_hint_dir(tmp_path_factory.mktemp("hints") / "h", (6, 10, 20), _rows(rng, 20_000), [_rows(rng, 7000)],
                         val_counts=counts, train_counts=[tuple(a[:7000] for a in counts)],
                         unigram_base=H.unigram(rng.integers(0, 50257, 1000)), val_tokens=20_000)
    return d


def test_device_rows_match_cpu_and_torch(hint_dir, monkeypatch):
    monkeypatch.setenv("HINT_NGRAM", "1")
    gpu, cpu = H.Hints(hint_dir, "cuda"), H.Hints(hint_dir, "cpu")
    rng = np.random.default_rng(0)
    # more lookups than ring slots, of growing and shrinking sizes (buffers regrown and reused), every index form
    lookups = [slice(0, 20_000), slice(5, 6), np.r_[np.arange(100, 900), np.arange(5000, 6000)],
               rng.permutation(20_000)[:4000], slice(19_000, 20_000), np.array([7, 3, 3, 19_999]), slice(0, 0)]
    for index in lookups * 2:
        g, c = gpu.val(index), cpu.val(index)
        assert g.cell.is_cuda and g.cell.dtype == torch.int64 and g.tokens.dtype == torch.int64
        assert torch.equal(g.cell.cpu(), c.cell) and torch.equal(g.tokens.cpu(), c.tokens)
        assert torch.equal(g.counts.cpu(), c.counts)
        # the reference's widening by torch on the GPU (division by the scalar): bit-exact
        raw = torch.from_numpy(np.asarray(gpu._val.a["weights"][index]).view(np.int16).copy()).cuda()
        assert torch.equal(g.weights, (raw.int() & 0xFFFF).float() / H.WEIGHT_ONE)
        assert torch.allclose(g.weights.cpu(), c.weights, rtol=1e-6, atol=0)
    t = gpu.train(0, np.arange(6000, 7000))
    assert torch.equal(t.cell.cpu(), cpu.train(0, np.arange(6000, 7000)).cell)
    assert torch.equal(t.counts.cpu(), cpu.train_span(0, 6000, 1000).counts)


def test_fake_rows_on_device(monkeypatch):
    monkeypatch.setenv("HINT_NGRAM", "1")
    monkeypatch.setenv("HINT_FAKE_SLOTS", "3")
    r = H.Hints("fake", "cuda").val(slice(0, 5000))
    assert r.cell.shape == (5000, 3) and r.counts.shape == (5000, 3, 10) and r.weights.is_cuda
    s = r.weights.sum(-1)
    assert torch.allclose(s[r.cell > 0], torch.ones_like(s[r.cell > 0]), atol=1e-4)


def test_val_stats_outputs_through_the_directory(tmp_path, monkeypatch):
    """The validation statistics' rows and counts, written as a hint directory and read back on the device."""
    corpus = data.make_corpus("c1", train_tokens=400_000, query_tokens=30_001, shard_tokens=200_000)
    tok, sizes, starts, L = data.device_tokens(corpus.shards())
    x, tgt, avail = G.val_queries(corpus.query)
    res = G.build_stats(tok, sizes, starts, x, tgt, avail)
    host = G.host_outputs(res)
    N = x.numel()
    v = 0  # the first variant (6, 10, 20)
    d = H.write_hint_dir(tmp_path / "h", G.VARIANTS[v], (host["cell"][v], host["tokens"][v], host["weights"][v]),
                         val_counts=(host["tot"], host["dist"], host["cnt"]), count_levels=G.ALL_LEVELS,
                         unigram_base=H.unigram(corpus.shards()[0]), val_tokens=N)
    monkeypatch.setenv("HINT_NGRAM", "1")
    r = H.Hints(d, "cuda").val_span(0, N)
    assert np.array_equal(r.cell.cpu().numpy(), host["cell"][v].astype(np.int64))
    assert np.array_equal(r.tokens.cpu().numpy(), host["tokens"][v].astype(np.int64))
    assert np.array_equal(np.rint(r.weights.cpu().numpy() * H.WEIGHT_ONE).astype(np.uint16), host["weights"][v])
    assert np.array_equal(r.counts[:, 0].cpu().numpy(), host["tot"].astype(np.float32))
    assert np.array_equal(r.counts[:, 2].cpu().numpy(), host["cnt"].astype(np.float32))
    assert (r.cell > 0).any()
