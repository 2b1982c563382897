"""GPU: the validation statistics' surface (ngram_amd.gpu_val_stats: build_stats, InProcess, the CLI; the surface of
old_records/gpu_val_stats.py) bit-exact against the CPU oracle on seeded synthetic streams: tot / dist / cnt per
position and level with the TOP = 1024 rule, and the variants' hint rows; the threaded shard loader against the
synchronous layout."""

import numpy as np
import pytest
import torch

import oracle as O
from ngram_amd import data
from ngram_amd import gpu_val_stats as G
from ngram_amd.loader import Loader

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def corpus():
    return data.make_corpus("c1", train_tokens=600_000, query_tokens=40_001, shard_tokens=250_000)


@pytest.fixture(scope="module")
def reference(corpus):
    x, tgt = corpus.query[:-1], corpus.query[1:]
    avail = O.segments(x)
    return {k: O.query_counts(corpus.train, corpus.bounds, x, tgt, avail, k) for k in G.ALL_LEVELS}


def _check(counts, rows, reference, levels, variants):
    counts = counts.cpu().numpy()
    for li, k in enumerate(levels):
        o = reference[k]
        assert np.array_equal(counts[0, li].view(np.uint32), o["tot"]), f"tot k={k}"
        assert np.array_equal(counts[1, li].astype(np.uint16), o["dist"]), f"dist k={k}"
        assert np.array_equal(counts[2, li].view(np.uint32), o["cnt"]), f"cnt k={k}"
        assert (o["tot"] > 0).sum() > 0
    rows = rows.cpu().numpy()
    for v, lv in enumerate(variants):
        cell, tokens, w = O.deepest_rows({k: reference[k] for k in lv}, lv)
        assert np.array_equal(rows[v], O.pack_rows(cell, tokens, w)), f"rows {lv}"


def test_build_stats_matches_oracle(gpu, corpus, reference):
    tok, sizes, starts, L = data.device_tokens(corpus.shards())
    x, tgt, avail = G.val_queries(corpus.query)
    res = G.build_stats(tok, sizes, starts, x, tgt, avail)
    _check(res["counts"], res["rows"], reference, G.ALL_LEVELS, G.VARIANTS)
    # the mask: bit li where the level's context occurred
    mask = res["mask"].cpu().numpy()
    for li, k in enumerate(G.ALL_LEVELS):
        assert np.array_equal((mask >> li) & 1, (reference[k]["tot"] > 0).astype(np.int32)), k


def test_top_rule_applies(gpu):
    """Context (7, 8) followed by 1500 distinct tokens, token 100 + t appearing 1 + (t % 3) times: ranked by count
    descending then token ascending, the count-3 tokens take ranks 0-499, the count-2 ones 500-999 and the count-1 ones
    (100, 103, ...) 1000-1499, so within TOP = 1024 only up to token 169 (rank 1023); 172 (rank 1024) gets cnt 0."""
    body = []
    for t in range(1500):
        body += [7, 8, 100 + t] * (1 + t % 3)
    train = np.array(body, np.uint16)
    q = np.array([7, 8, 100, 7, 8, 172, 7, 8, 102, 7, 8, 169, 7, 8, 1598], np.uint16)
    tok, sizes, starts, L = data.device_tokens([train])
    x, tgt, avail = G.val_queries(q)
    res = G.build_stats(tok, sizes, starts, x, tgt, avail, levels=(2, 3), variants=((2, 3),))
    got = res["counts"][2, 0].cpu().numpy().view(np.uint32)
    assert got[[1, 4, 7, 10, 13]].tolist() == [1, 0, 3, 1, 2]
    want = O.query_counts(train, np.array([0, len(train)]), q[:-1], q[1:], O.segments(q[:-1]), 2)
    assert np.array_equal(got, want["cnt"])
    assert res["counts"][1, 0].cpu().numpy()[1] == 1500 and res["counts"][0, 0].cpu().numpy()[1] == 3000


def test_loader_matches_device_tokens(gpu, corpus, tmp_path):
    """Chunks far smaller than a shard (workers share a shard), more workers than shards, an empty shard: the buffer
    equals the synchronous layout; the per-shard events order a consumer after each shard's copies."""
    shards = corpus.shards() + [np.zeros(0, np.uint16)]
    paths = []
    for i, s in enumerate(shards):
        p = tmp_path / f"s{i}.bin"
        data.write_shard(p, s)
        paths.append(str(p))
    want, sizes, starts, L = data.device_tokens(shards)
    for threads, chunk in ((1, 70_001), (3, 4096), (5, 1 << 20)):
        ld = Loader(paths, L, starts, sizes, threads, chunk_tokens=chunk)
        ev = ld.shard_events()
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            for i in range(len(ev)):
                s.wait_event(ev[i])
            got = ld.tok.clone()
        s.synchronize()
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


def test_loader_copies_follow_the_fill(gpu, corpus, tmp_path):
    """The buffer's SENT fill is queued behind a long kernel on the constructing thread's stream; the workers' copies
    (on their own streams) still land after it, not under it."""
    shards = corpus.shards()
    paths = []
    for i, s in enumerate(shards):
        p = tmp_path / f"f{i}.bin"
        data.write_shard(p, s)
        paths.append(str(p))
    want, sizes, starts, L = data.device_tokens(shards)
    torch.cuda.synchronize()
    torch.cuda._sleep(200_000_000)  # keeps the current stream busy for a while
    ld = Loader(paths, L, starts, sizes, 4, chunk_tokens=1 << 16)
    ld.wait_all()
    got = ld.tok.clone()
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    ld.join()


@pytest.mark.parametrize("background", [False, True])
def test_in_process_loads_and_builds(gpu, corpus, reference, tmp_path, background):
    """InProcess: the shards loaded by the threaded loader while the query index is built, each shard's first scan
    waiting for its copy, on the caller's thread or a background one; outputs equal the oracle's."""
    paths, val_path = corpus.write(tmp_path)
    n = len(corpus.query) - 1
    ip = G.InProcess(paths, val_path, variants=G.VARIANTS, threads=3, chunk_mb=1, val_tokens=n)
    ip.prepare()
    if background:
        ip.start_background()
    else:
        ip.start_load()
    res = ip.finish()
    _check(res["counts"], res["rows"], reference, G.ALL_LEVELS, G.VARIANTS)
    assert res["timing"]["load"]["bytes"] == 2 * len(corpus.train)


def test_cli_writes_the_reference_layout(gpu, corpus, reference, tmp_path):
    paths, val_path = corpus.write(tmp_path / "in")
    lst = tmp_path / "shards.txt"
    lst.write_text("\n".join(paths))
    n = len(corpus.query) - 1
    out = tmp_path / "out"
    G.run(G.parse_args(["--shards", str(lst), "--val", val_path, "--out", str(out), "--threads", "2",
                        "--val-tokens", str(n), "--fused", "--direct"]))
    tot, dist, cnt = (np.load(out / f"{name}.npy") for name in ("tot", "dist", "cnt"))
    assert tot.dtype == np.uint32 and dist.dtype == np.uint16 and cnt.dtype == np.uint32
    for li, k in enumerate(G.ALL_LEVELS):
        assert np.array_equal(tot[:, li], reference[k]["tot"]) and np.array_equal(dist[:, li], reference[k]["dist"])
        assert np.array_equal(cnt[:, li], reference[k]["cnt"]), k
    for lv in G.VARIANTS:
        d = out / ("rows_" + "_".join(map(str, lv)))
        cell, tokens, w = O.deepest_rows({k: reference[k] for k in lv}, lv)
        assert np.array_equal(np.load(d / "cell.npy"), cell.astype(np.int16))
        assert np.array_equal(np.load(d / "tokens.npy"), tokens)
        assert np.array_equal(np.load(d / "weights.npy"), w)
