"""GPU: the gpu_val_stats path (our C ABI + the host mirror) bit-exact against the CPU oracle on seeded synthetic
streams: tot / dist / cnt per position and level, and the variants' hint rows."""

import numpy as np
import pytest
import torch

import oracle as O
from ngram_amd import data
from ngram_amd import gpu_val_stats as G

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def corpus():
    return data.make_corpus("c1", train_tokens=600_000, query_tokens=40_001, shard_tokens=250_000)


@pytest.fixture(scope="module")
def reference(corpus):
    x, tgt = corpus.query[:-1], corpus.query[1:]
    avail = O.segments(x)
    return {k: O.query_counts(corpus.train, corpus.bounds, x, tgt, avail, k) for k in G.ALL_LEVELS}


def _check(res, reference, levels, variants):
    counts = res["counts"].cpu().numpy()
    for li, k in enumerate(levels):
        o = reference[k]
        assert np.array_equal(counts[0, li].view(np.uint32), o["tot"]), f"tot k={k}"
        assert np.array_equal(counts[1, li].astype(np.uint16), o["dist"]), f"dist k={k}"
        assert np.array_equal(counts[2, li].view(np.uint32), o["cnt"]), f"cnt k={k}"
        assert (o["tot"] > 0).sum() > 0
    rows = res["rows"].cpu().numpy()
    for v, lv in enumerate(variants):
        cell, tokens, w = O.deepest_rows({k: reference[k] for k in lv}, lv)
        assert np.array_equal(rows[v], O.pack_rows(cell, tokens, w)), f"rows {lv}"


@pytest.mark.parametrize("mode", ["partitioned", "direct", "fused", "words"])
def test_build_stats_matches_oracle(lib, corpus, reference, mode):
    tok, sizes, starts, L = G.load_shards(corpus.shards())
    x, tgt, avail = G.query_tensors(corpus.query)
    kw = dict(direct=mode == "direct", fused=mode == "fused", words_density=4.0 if mode == "words" else 0.0)
    res = G.build_stats(lib, tok, L, starts, sizes, x, tgt, avail, **kw)
    _check(res, reference, G.ALL_LEVELS, G.VARIANTS)


def test_val_index_is_canonical(lib, corpus):
    x, tgt, avail = G.query_tensors(corpus.query)
    vi = G.ValIndex(lib, x, avail, 3)
    table = vi.table.cpu().numpy().view(np.uint64)
    occupied = table != np.uint64(2 ** 64 - 1)
    assert occupied.sum() == vi.n and not occupied[-1]
    keys = table[occupied]
    assert np.all(np.diff(keys.astype(np.float64)) >= 0)  # ascending keys = ascending home slots
    ctx = vi.ctx_of.cpu().numpy()
    av = avail.cpu().numpy()
    assert np.all((ctx >= 0) == (av >= 3))


def test_overflow_reruns_with_a_bigger_table(lib, corpus, reference):
    # a pair table far too small for level 2 overflows (flags[0]); the level reruns with twice the slots
    tok, sizes, starts, L = G.load_shards(corpus.shards())
    x, tgt, avail = G.query_tensors(corpus.query)
    old = G.LOAD
    try:
        G.LOAD = 1e9  # the estimates shrink to nothing: a 1024-slot table
        res = G.build_stats(lib, tok, L, starts, sizes, x, tgt, avail, levels=(2, 3), variants=((2, 3),),
                            min_cap=1024)
    finally:
        G.LOAD = old
    assert res["levels"][2]["reruns"] > 0
    _check(res, reference, (2, 3), ((2, 3),))


def test_loader_matches_load_shards(corpus, tmp_path):
    """Threaded pread into pinned staging buffers: chunks far smaller than a shard (each thread's two buffers reused
    many times), more threads than some shards get, and an empty shard; the buffer equals the synchronous layout."""
    from ngram_amd.loader import Loader

    shards = corpus.shards() + [np.zeros(0, np.uint16)]
    paths = []
    for i, s in enumerate(shards):
        p = tmp_path / f"s{i}.bin"
        data.write_shard(p, s)
        paths.append(str(p))
    want, sizes, starts, L = G.load_shards(shards)
    for threads, chunk in ((1, 70_001), (2, 4096), (5, 1 << 20)):
        ld = Loader(paths, L, starts, sizes, threads, chunk_tokens=chunk)
        got = ld.tok
        ld.wait_all()
        assert torch.equal(got, want), (threads, chunk)
        ld.join()
        assert ld.stats["seconds"] >= 0 and ld.stats["bytes"] == 2 * sum(sizes)
    with pytest.raises(ValueError):
        Loader(paths, L, starts, sizes, 2, mode="register")
    ld = Loader(paths, L, starts, sizes, 2, start=False)
    with pytest.raises(ValueError):
        ld.wait(0)  # not started
    with pytest.raises(ValueError):
        ld.start(stream_priority=-1)
    ld = Loader([str(tmp_path / "missing.bin")], L, starts[:1], sizes[:1], 1)
    with pytest.raises(FileNotFoundError):
        ld.wait(0)


@pytest.mark.parametrize("background", [False, True])
def test_in_process_loads_and_builds(corpus, reference, tmp_path, background):
    """InProcess: the shards loaded by the threaded loader while the query index is built, each shard scanned once
    its copy lands (fused and per-level), on the caller's thread or a background one; outputs equal the oracle's."""
    paths, val_path = corpus.write(tmp_path)
    n = len(corpus.query) - 1
    flags = ("--fused", "--direct") if background else ("--direct",)
    ip = G.InProcess(paths, val_path, variants=G.VARIANTS, threads=3, chunk_mb=1, flags=flags, val_tokens=n)
    ip.prepare()
    if background:
        ip.start_background()
    else:
        ip.start_load()
    res = ip.finish()
    _check(res, reference, G.ALL_LEVELS, G.VARIANTS)
    assert res["timing"]["load"]["bytes"] == 2 * len(corpus.train)
