"""Validation-side exact n-gram statistics on one MI355X, with the surface of old_records/gpu_val_stats.py: the CLI
(flags :657-681, outputs :1216-1228), `InProcess` (:1235-1316: prepare / start_load / start_background / finish), the
constants (ALL_LEVELS, LEVELS, VARIANTS, TOP, ENTRIES, VAL_TOKENS) and the output layout; computed by the engine's level
pipeline (levels.LevelBuild) instead of the reference's per-level hash tables and ranking sorts.

Outputs, as the reference's: `counts` int32 [3, len(ALL_LEVELS), N] -- per validation position and level its
k-context's total occurrences tot (uint32 bits), its distinct next tokens dist (at most 65535) and cnt, the count of the
position's own next token if it ranks among the context's TOP = 1024 most frequent (count descending, token
ascending), else 0 -- and `rows` int32 [len(variants), N, 9], per variant the hint row of the deepest of its levels
whose context occurred: cell, the 8 top next tokens two per int32, their weights two per int32 (ng_variant_rows). The
CLI saves tot / dist / cnt.npy [N, 10] (uint32 / uint16 / uint32) and rows_<levels>/{cell, tokens, weights}.npy.

One GPU: the reference's multi-GPU flags (--ipc, --async-init, --nccl-warmup, --own-device, --pipeline) are accepted
and change nothing; so are its counting strategies (--direct, --fused, --words-density, --chunk-positions), since
every level here is counted by the one partitioned path."""

from __future__ import annotations

import argparse
import json
import threading
import time
from pathlib import Path

import numpy as np
import torch

from . import data
from .lib import Lib, i32
from .levels import LevelBuild
from .loader import Loader

ALL_LEVELS = (2, 3, 4, 5, 6, 8, 10, 12, 16, 20)
LEVELS = (2, 3, 4, 5, 6, 10, 20)  # the hint rows' levels (a cell's length bucket is the index here)
VARIANTS = ((6, 10, 20), (2, 3, 6, 10, 20), LEVELS)
VAL_TOKENS = 10_485_760
TOP = 1024
ENTRIES = 8


def val_queries(val: np.ndarray, n: int | None = None, device="cuda"):
    """x, tgt, avail of the validation stream (its first n positions' inputs, then one more token): int16, int16,
    int32 on the device; avail = the position's tokens since its segment's start (a BOS starts one)."""
    val = np.asarray(val, np.uint16)
    N = len(val) - 1 if n is None else min(n, len(val) - 1)
    x = val[:N]
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    return to(x.view(np.int16)), to(val[1 : N + 1].view(np.int16)), to(data.segments(x))


def build_stats(tok: torch.Tensor, sizes: list[int], starts: list[int], x: torch.Tensor, tgt: torch.Tensor,
                avail: torch.Tensor, *, levels=ALL_LEVELS, variants=VARIANTS, ready: list | None = None,
                engine: LevelBuild | None = None, lib: Lib | None = None) -> dict:
    """The statistics of the query positions (x, tgt, avail) over the shards in `tok` (data.pack_layout's sizes and
    starts). `ready`: per shard an event its first scan waits for (e.g. Loader.wait(i)), or None for resident tokens.
    `engine`: a LevelBuild of these inputs from an earlier call (its sizing carries over). Returns {"counts", "rows",
    "levels" (per-level sizes), "mask" (bit li: level li's context occurred)}."""
    if not all(set(v) <= set(LEVELS) and set(v) <= set(levels) for v in variants):
        raise ValueError(f"variants {variants} must be of {LEVELS} and of the counted levels")
    lib = lib or Lib()
    eng = engine or LevelBuild(tok, sizes, starts, levels, ready=ready, elib=lib)
    keep = sorted({k for v in variants for k in v})
    res = eng.build(x, tgt, avail, cnt_top=TOP, keep=keep, with_mask=True)
    N = x.numel()
    rows = torch.zeros((len(variants), N, 9), dtype=torch.int32, device=x.device)
    for v, lv in enumerate(variants):
        desc = []
        for k in lv:
            ctx_of, rec = res.kept[k]
            desc += [eng.levels.index(k), LEVELS.index(k), ctx_of.data_ptr(), rec.data_ptr()]
        d = torch.tensor(desc, dtype=torch.int64, device=x.device)
        lib("ng_variant_rows", N, res.mask, i32(len(lv)), d, rows[v])
    torch.cuda.current_stream().synchronize()  # the descriptors' records are freed with `res`
    return {"counts": res.counts, "rows": rows, "levels": res.info, "mask": res.mask}


def host_outputs(result: dict) -> dict[str, np.ndarray]:
    """The CLI's arrays: tot / dist / cnt [N, L], cell [V, N], tokens / weights [V, N, 8]."""
    c, rows = result["counts"], result["rows"]
    h = lambda t: t.contiguous().cpu().numpy()  # noqa: E731
    return {"tot": h(c[0].t()).view(np.uint32), "dist": h(c[1].t().to(torch.int16)).view(np.uint16),
            "cnt": h(c[2].t()).view(np.uint32), "cell": h(rows[:, :, 0].to(torch.int16)),
            "tokens": h(rows[:, :, 1:5]).view(np.uint16), "weights": h(rows[:, :, 5:9]).view(np.uint16)}


def save_outputs(out: Path, result: dict, variants=VARIANTS) -> None:
    """tot.npy, dist.npy, cnt.npy and rows_<levels>/{cell, tokens, weights}.npy in `out`."""
    out.mkdir(parents=True, exist_ok=True)
    h = host_outputs(result)
    for name in ("tot", "dist", "cnt"):
        np.save(out / f"{name}.npy", h[name])
    for v, lv in enumerate(variants):
        d = out / ("rows_" + "_".join(map(str, lv)))
        d.mkdir(exist_ok=True)
        for name in ("cell", "tokens", "weights"):
            np.save(d / f"{name}.npy", h[name][v])


def parse_args(argv: list[str] | None = None) -> argparse.Namespace:
    """The reference's flags (old_records/gpu_val_stats.py:657-681), plus --val-tokens."""
    ap = argparse.ArgumentParser(description="exact n-gram statistics of the validation positions on one GPU")
    ap.add_argument("--shards", required=True, help="a file listing the training shard paths")
    ap.add_argument("--val", required=True, help="the validation shard file")
    ap.add_argument("--out", required=True, help="the output directory")
    ap.add_argument("--threads", type=int, default=8, help="loader threads")
    ap.add_argument("--load-mode", choices=("register", "pread"), default="pread")
    ap.add_argument("--chunk-mb", type=int, default=16, help="the loader's staging buffers (MB)")
    ap.add_argument("--sequential", action="store_true", help="load every shard before the build starts")
    ap.add_argument("--numa", action="store_true", help="loader threads on the GPU's NUMA node")
    for flag in ("--direct", "--pipeline", "--async-init", "--nccl-warmup", "--own-device", "--ipc", "--early-ctx",
                 "--fused", "--bench-io"):
        ap.add_argument(flag, action="store_true", help="accepted; no effect on one GPU")
    ap.add_argument("--words-density", type=float, default=0.0, help="accepted; no effect")
    ap.add_argument("--chunk-positions", type=int, default=0, help="accepted; no effect")
    ap.add_argument("--no-save", action="store_true")
    ap.add_argument("--val-tokens", type=int, default=VAL_TOKENS, help="validation positions")
    ap.add_argument("--launch-time", type=float, default=float("nan"))
    return ap.parse_args(argv)


def _read_val(path: str, n: int) -> np.ndarray:
    v = data.read_shard(path)
    return np.array(v[: min(len(v), n + 1)])


def run(args: argparse.Namespace, variants=VARIANTS) -> dict:
    """main()'s build: shards from the listed files (loaded while the query index is built), the validation shard,
    outputs saved to args.out unless --no-save. Returns the result with its timing."""
    t0 = time.time()
    paths = [p for p in Path(args.shards).read_text().split() if p]
    sizes = [data.shard_tokens(p) for p in paths]
    starts, L = data.pack_layout(sizes)
    loader = Loader(paths, L, starts, sizes, args.threads, args.load_mode, args.chunk_mb << 19, args.numa)
    if args.sequential:
        loader.wait_all()
    x, tgt, avail = val_queries(_read_val(args.val, args.val_tokens), args.val_tokens)
    ready = None if args.sequential else loader.shard_events()
    res = build_stats(loader.tok, sizes, starts, x, tgt, avail, variants=variants, ready=ready)
    loader.join()
    res["timing"] = {"total_s": time.time() - t0, "load": {"seconds": loader.stats["seconds"],
                                                           "bytes": loader.stats["bytes"], "threads": args.threads}}
    if not args.no_save:
        out = Path(args.out)
        save_outputs(out, res, variants)
        (out / "timings.json").write_text(json.dumps([res["timing"]], indent=1))
    return res


def main() -> None:
    run(parse_args())


class InProcess:
    """The build inside a process that holds the GPU (the reference's InProcess, one GPU):
      - construct (before the clock): the shards' layout, the token buffer and the loader's pinned buffers allocated;
      - prepare() (before the clock): nothing to connect on one GPU;
      - start_load() (optional, on the clock): the shards' loads start in background threads;
      - start_background() (optional, instead): the loads and the whole build on a background thread and stream;
      - finish(): the build (each shard's first scan waits for that shard's copy), or the background build's result:
        {"counts": int32 [3, len(ALL_LEVELS), N], "rows": int32 [len(variants), N, 9], "timing"}.
    `variants`: the hint rows' level sets (each of LEVELS); `flags`: CLI flags (see parse_args)."""

    def __init__(self, shard_paths: list[str], val_path: str, variants=(LEVELS,), threads: int = 12, chunk_mb: int = 16,
                 flags: tuple[str, ...] = ("--fused", "--direct"), val_tokens: int = VAL_TOKENS):
        self.variants = tuple(tuple(v) for v in variants)
        if not all(set(v) <= set(LEVELS) for v in self.variants):
            raise ValueError(f"variants {self.variants} must be of {LEVELS}")
        self.args = parse_args(["--shards", "-", "--val", val_path, "--out", "-", "--threads", str(threads),
                                "--chunk-mb", str(chunk_mb), "--val-tokens", str(val_tokens), *flags])
        self.paths = list(shard_paths)
        self.sizes = [data.shard_tokens(p) for p in self.paths]
        self.starts, self.L = data.pack_layout(self.sizes)
        self.device = torch.cuda.current_device()
        self.loader = Loader(self.paths, self.L, self.starts, self.sizes, threads, "pread", chunk_mb << 19, start=False)
        self.loader.preallocate()
        self.lib = Lib()
        self.thread = self.error = self.result = None

    def prepare(self) -> None:
        torch.cuda.synchronize()

    def start_load(self) -> None:
        if not self.loader.started:
            self.loader.start()

    def start_background(self) -> None:
        """The loads and the build from now, on a background thread and a stream of its own; finish() returns it."""
        if self.thread is not None:
            raise ValueError("the build has already started")
        self.start_load()
        stream = torch.cuda.Stream(device=self.device)

        def work() -> None:
            try:
                torch.cuda.set_device(self.device)
                with torch.cuda.stream(stream):
                    self.result = self._build()
                stream.synchronize()
            except BaseException as e:  # noqa: BLE001 - raised again by finish()
                self.error = e

        self.thread = threading.Thread(target=work, daemon=True)
        self.thread.start()

    def _build(self) -> dict:
        t0 = time.time()
        x, tgt, avail = val_queries(_read_val(self.args.val, self.args.val_tokens), self.args.val_tokens)
        res = build_stats(self.loader.tok, self.sizes, self.starts, x, tgt, avail, variants=self.variants,
                          ready=self.loader.shard_events(), lib=self.lib)
        self.loader.join()
        timing = {"total_s": time.time() - t0, "levels": res["levels"],
                  "load": {"seconds": self.loader.stats["seconds"], "bytes": self.loader.stats["bytes"]}}
        return {"counts": res["counts"], "rows": res["rows"], "timing": timing}

    def finish(self) -> dict:
        if self.thread is None:
            self.start_load()
            return self._build()
        t0 = time.time()
        self.thread.join()
        self.waited = time.time() - t0
        if self.error is not None:
            raise self.error
        torch.cuda.current_stream().synchronize()
        return self.result


if __name__ == "__main__":
    main()
