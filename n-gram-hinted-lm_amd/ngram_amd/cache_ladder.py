"""A GPU rung for cache_ladder's build-speed ladder (cache_ladder/src/lib.rs:1-8, cache_ladder.pyi): the ladder's
indexes all build, from the first `tokens` tokens of the training shards, the record's 6/10/20-gram -> next-token
cache, with the interface `create(files, tokens, threads, cpus)` (before the clock: open the shards, load them) and
`build() -> dict` (the timed part, returning statistics of what it built). `GpuCountIndex` builds that cache exactly
on the GPU: the CountTable of every 6-, 10- and 20-token context of those tokens (count_table.py), each context's
total, distinct next tokens and top next tokens. The CPU rungs' approximations (next tokens capped per context,
fingerprint buckets) are not reproduced: this rung is exact."""

from __future__ import annotations

import os
import time

import numpy as np
import torch

from .count_table import CountTable
from .data import HEADER_BYTES, shard_tokens

LEVELS = (6, 10, 20)


class GpuCountIndex:
    def __init__(self):
        raise TypeError("use GpuCountIndex.create(files, tokens, threads, cpus)")

    @staticmethod
    def create(files: list[str], tokens: int, threads: int = 1, cpus: list[int] = ()) -> "GpuCountIndex":
        """The shards holding the first `tokens` tokens, the last one cut to fit, read into GPU memory; ValueError if
        the files hold fewer or a shard is invalid (lib.rs shards :47-82)."""
        arrays, left = [], int(tokens)
        for f in files:
            if left == 0:
                break
            n = shard_tokens(f) if isinstance(f, (str, bytes, os.PathLike)) else len(f)
            a = (np.fromfile(f, dtype="<u2", count=n, offset=HEADER_BYTES)
                 if isinstance(f, (str, bytes, os.PathLike)) else np.ascontiguousarray(f, dtype=np.uint16))
            a = a[: min(n, left)]
            left -= len(a)
            arrays.append(a)
        if left > 0:
            raise ValueError(f"the files hold {tokens - left} tokens, fewer than {tokens}")
        self = object.__new__(GpuCountIndex)
        self.table = CountTable.create(arrays, list(LEVELS), max(1, threads), list(cpus))
        self.tokens = int(tokens)
        return self

    def build(self) -> dict[str, float]:
        """The timed build: every level's exact table. Returns seconds, tokens, and per level its contexts, pairs and
        bytes."""
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        self.table.build()
        torch.cuda.synchronize()
        out = {"seconds": time.perf_counter() - t0, "tokens": float(self.tokens)}
        for k, contexts, pairs, nbytes in self.table.sizes():
            out[f"contexts_{k}"] = float(contexts)
            out[f"pairs_{k}"] = float(pairs)
            out[f"bytes_{k}"] = float(nbytes)
        return out
