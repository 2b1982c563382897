"""CPU: the hint directory (ngram_amd.hints, the format of old_records/hint_runtime.py): the writer's layout and
checks, the reader's lookups on device="cpu" (slices, runs of positions, scattered positions, count rows, slots), the
weights against the oracle's restatement of old_records.py's _weights and known answers, the fake rows'
invariants."""

import json

import numpy as np
import pytest
import torch

import oracle as O
from ngram_amd import hints as H


def _rows(rng, n, slots=1, entries=8):
    lead = (n,) if slots == 1 else (n, slots)
    hinted = rng.random(lead) < 0.6
    cell = np.where(hinted, rng.integers(1, 336, lead), 0).astype(np.int16)
    counts = np.sort(rng.integers(0, 50, (*lead, entries)), -1)[..., ::-1] * hinted[..., None]
    tokens = rng.integers(0, 50257, (*lead, entries)).astype(np.uint16)
    return cell, tokens, H.weights(counts)


def _counts(rng, n, L):
    tot = rng.integers(0, 1 << 31, (n, L)).astype(np.uint32)
    dist = np.minimum(tot, rng.integers(0, 65536, (n, L))).astype(np.uint16)
    cnt = (rng.random((n, L)) * tot).astype(np.uint32)
    return tot, dist, cnt


def test_weights_known_answers_and_oracle():
    # half to even: 1/2 of 65535 = 32767.5 -> 32768; 3/4 -> 49151.25 -> 49151, 1/4 -> 16383.75 -> 16384
    got = H.weights(np.array([[1, 1, 0], [3, 1, 0], [0, 0, 0], [7, 0, 0]]))
    assert got.tolist() == [[32768, 32768, 0], [49151, 16384, 0], [0, 0, 0], [65535, 0, 0]]
    c = np.random.default_rng(1).integers(0, 1 << 20, (1000, 8)) * (np.arange(8) < 5)
    assert np.array_equal(H.weights(c), O.weights(c))
    u = H.unigram(np.array([0, 0, 50256], np.uint16))
    assert u.dtype == np.float32 and u.shape == (H.VOCAB,) and abs(float(u.sum()) - 1) < 1e-5
    assert u[0] == np.float32(2.5 / (3 + 0.5 * H.VOCAB)) and u[1] == np.float32(0.5 / (3 + 0.5 * H.VOCAB))


def test_write_and_read_cpu(tmp_path, monkeypatch):
    rng = np.random.default_rng(0)
    L = len(H.FAKE_COUNT_LEVELS)
    val, train = _rows(rng, 5000), [_rows(rng, 3000), _rows(rng, 100)]
    vc, tc = _counts(rng, 5000, L), [_counts(rng, 3000, L)]
    d = H.write_hint_dir(tmp_path / "h", (6, 10, 20), val, train, val_counts=vc, train_counts=tc,
                         unigram_base=H.unigram(rng.integers(0, 50257, 1000)), val_tokens=5000)
    meta = json.loads((d / "meta.json").read_text())
    assert meta == {"levels": [6, 10, 20], "cells": 336, "entries": 8, "train_shards": 2, "val_tokens": 5000,
                    "slots": 1, "buckets": list(H.BUCKETS), "count_levels": list(H.FAKE_COUNT_LEVELS),
                    "count_shards": 1}
    assert np.load(d / "train" / "0001" / "cell.npy").dtype == np.int16
    monkeypatch.setenv("HINT_NGRAM", "1")
    h = H.Hints(d, device="cpu")
    assert h.cells == 336 and h.levels == (6, 10, 20) and h.count_levels == H.FAKE_COUNT_LEVELS
    runs = np.r_[np.arange(10, 400), np.arange(1000, 1700)]  # two runs: copied run by run
    scattered = rng.permutation(5000)[:300]
    for index in (slice(0, 5000), slice(17, 1017), runs, scattered, np.array([], np.int64)):
        r = h.val(index)
        c, t, w = (a[index] for a in val)
        assert r.cell.dtype == torch.int64 and np.array_equal(r.cell.numpy(), c)
        assert np.array_equal(r.tokens.numpy(), t.astype(np.int64))
        assert r.weights.dtype == torch.float32
        assert np.allclose(r.weights.numpy(), w / 65535, rtol=1e-6, atol=0)
        assert np.array_equal(r.counts.numpy(), np.stack([a[index] for a in vc], 1).astype(np.float32))
    hinted = val[0] > 0
    assert np.allclose(h.val(slice(0, 5000)).weights.numpy()[hinted].sum(-1), 1, atol=1e-4)
    r = h.train(0, slice(100, 200))
    assert np.array_equal(r.tokens.numpy(), train[0][1][100:200].astype(np.int64))
    assert np.array_equal(h.train_span(0, 100, 100).cell.numpy(), r.cell.numpy())
    with pytest.raises(IndexError):
        h.val(slice(0, 5001))
    with pytest.raises(IndexError):
        h.val(np.array([5000]))
    with pytest.raises(IndexError):
        h.train(2, slice(0, 1))
    with pytest.raises(IndexError):
        h.train(1, slice(0, 1))  # shard 1 has hint rows, no count rows
    monkeypatch.setenv("HINT_NGRAM", "0")
    assert H.Hints(d, device="cpu").train(1, slice(0, 100)).counts is None


def test_slots_and_errors(tmp_path, monkeypatch):
    rng = np.random.default_rng(2)
    val = _rows(rng, 800, slots=3)
    d = H.write_hint_dir(tmp_path / "s", (2, 6), val, slots=3, val_tokens=800)
    r = H.Hints(d, device="cpu").val(np.arange(100, 300))
    assert r.cell.shape == (200, 3) and r.tokens.shape == (200, 3, 8) and r.weights.shape == (200, 3, 8)
    assert np.array_equal(r.cell.numpy(), val[0][100:300])
    with pytest.raises(ValueError):
        H.write_hint_dir(tmp_path / "e1", (6, 7), val, slots=3)  # 7 is not a bucket
    with pytest.raises(ValueError):
        H.write_hint_dir(tmp_path / "e2", (6,), val)  # slot axis where one slot is declared
    with pytest.raises(ValueError):
        H.write_hint_dir(tmp_path / "e3", (6,), _rows(rng, 10), val_counts=_counts(rng, 10, 10))  # no unigram
    monkeypatch.setenv("HINT_NGRAM", "1")
    with pytest.raises(ValueError):
        H.Hints(d, device="cpu")  # no count rows


def test_fake_rows(monkeypatch):
    monkeypatch.setenv("HINT_NGRAM", "1")
    monkeypatch.setenv("HINT_FAKE_SLOTS", "2")
    h = H.Hints("fake", device="cpu")
    r = h.val(slice(0, 4000))
    assert r.cell.shape == (4000, 2) and r.tokens.shape == (4000, 2, 8)
    hinted = (r.cell > 0).numpy()
    s = r.weights.sum(-1).numpy()
    assert 0.3 < hinted.mean() < 0.7 and np.allclose(s[hinted], 1, atol=1e-4) and np.all(s[~hinted] == 0)
    c = r.counts.numpy()
    tot, dist, cnt = c[:, 0], c[:, 1], c[:, 2]
    assert c.shape == (4000, 3, 10) and np.all(np.diff(tot, axis=1) <= 0)
    assert np.all(dist <= tot) and np.all(cnt <= tot) and (tot[:, 0] > 0).mean() > 0.8
    with pytest.raises(IndexError):
        h.val(slice(H.VAL_TOKENS, H.VAL_TOKENS + 1))


def test_cpulist_parsing():
    """The loader's NUMA pinning reads sysfs CPU lists: ranges, single CPUs, a trailing newline, an empty list."""
    from ngram_amd.loader import _cpulist

    assert _cpulist("0-3,8,10-11\n") == {0, 1, 2, 3, 8, 10, 11}
    assert _cpulist("5") == {5} and _cpulist("") == set()
