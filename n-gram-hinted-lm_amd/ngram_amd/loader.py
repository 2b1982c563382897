"""Shard files into one device token buffer in background threads: the host data path of the validation statistics
(what old_records/gpu_val_stats.py's Loader :226-359 provides to its build: every shard copied to its place in a
GPU buffer laid out with SENT gaps, a per-shard event the first scan of that shard waits for, and the copies overlapping
the query index and the earlier shards' scans).

Design. The shards are cut into chunks of `chunk_tokens`, queued in shard order, and `threads` workers take chunks
from the one queue, so a large shard is read by every worker at once and the first shards complete first. A worker
reads its chunk with os.preadv (the GIL is released during the read) into one of its two pinned staging buffers and
enqueues the chunk's host-to-device copy on its own stream; it reuses a buffer once that buffer's previous copy has
completed, so it reads the next chunk while the last one crosses PCIe. A shard is complete when all its chunks are:
the worker that enqueues a shard's last chunk makes its stream wait for the shard's other chunks' copies and records
the shard's event there. Every copy waits for the buffer's initial SENT fill (recorded on the constructing thread's
stream), so a copy never races with it.

Platform notes: the mode "register" (pinning a shard's mapping in place with cudaHostRegister) raises ValueError,
since this platform refuses hipHostRegister of existing memory; the streams keep the default priority (`start`
refuses another), since work on streams of other priorities has hung on this platform."""

from __future__ import annotations

import os
import queue
import threading
import time
from pathlib import Path

import torch

from .data import HEADER_BYTES


def _cpulist(text: str) -> set[int]:
    """A sysfs CPU list ("0-3,8,10-11") as a set."""
    out: set[int] = set()
    for item in filter(None, text.strip().split(",")):
        ends = [int(v) for v in item.split("-")]
        out.update(range(ends[0], ends[-1] + 1))
    return out


def numa_cpus(device: int) -> set[int]:
    """The CPUs of the GPU's NUMA node that this process may use; empty when the topology is unknown (sysfs: the
    device's PCI function's numa_node, then that node's cpulist)."""
    try:
        props = torch.cuda.get_device_properties(device)
        pci = Path("/sys/bus/pci/devices") / "{:04x}:{:02x}:{:02x}.0".format(
            props.pci_domain_id, props.pci_bus_id, props.pci_device_id)
        node = int((pci / "numa_node").read_text())
        mine = os.sched_getaffinity(0)
        return set() if node < 0 else _cpulist(Path(f"/sys/devices/system/node/node{node}/cpulist").read_text()) & mine
    except (OSError, ValueError, AttributeError):
        return set()


class Loader:
    """Shards `paths` (sizes[i] tokens at starts[i]) into `tok` (a new int16 [tok_len] device buffer of SENT = -1,
    unless given), by `threads` workers started at construction unless `start` is False. `chunk_tokens`: the staging
    buffers' size (two per worker). `numa`: run the workers on the GPU's NUMA node. `stats`: bytes, per-worker read and
    enqueue seconds, the pinned allocation's seconds and, after join(), the seconds from start to the last copy."""

    def __init__(self, paths: list, tok_len: int, starts: list[int], sizes: list[int], threads: int,
                 mode: str = "pread", chunk_tokens: int = 8 << 20, numa: bool = False, start: bool = True,
                 tok: torch.Tensor | None = None):
        if mode != "pread":
            raise ValueError(f"load mode {mode!r}: only 'pread' (this platform refuses to pin existing memory in place)")
        if not len(paths) == len(starts) == len(sizes):
            raise ValueError("paths, starts and sizes need one entry per shard")
        if threads < 1 or chunk_tokens < 1:
            raise ValueError(f"threads ({threads}) and chunk_tokens ({chunk_tokens}) must be at least 1")
        if any(st < 0 or st + n > tok_len for st, n in zip(starts, sizes)):
            raise ValueError(f"a shard lies outside the buffer of {tok_len} tokens")
        self.paths, self.starts, self.sizes = [str(p) for p in paths], list(starts), list(sizes)
        self.tok = torch.full((tok_len,), -1, dtype=torch.int16, device="cuda") if tok is None else tok
        if self.tok.dtype != torch.int16 or self.tok.numel() < tok_len:
            raise ValueError("tok must be an int16 tensor of at least tok_len tokens")
        self.device = torch.cuda.current_device()
        self.filled = torch.cuda.Event()
        self.filled.record()  # on the constructing thread's stream, after the fill (or the caller's own writes)
        self.chunk_tokens, self.nworkers = chunk_tokens, threads
        self.cpus = numa_cpus(self.device) if numa else set()
        self.events: list = [None] * len(self.paths)
        self.ready = [threading.Event() for _ in self.paths]
        self.left = [max(1, -(-n // chunk_tokens)) for n in self.sizes]  # chunks per shard (an empty shard: one)
        self.chunk_events: list[list] = [[] for _ in self.paths]
        self.buffers: list = [None] * threads
        self.errors: list[BaseException] = []
        self.lock = threading.Lock()
        self.work: queue.SimpleQueue = queue.SimpleQueue()
        self.stats = {"mode": mode, "threads": threads, "bytes": 2 * sum(self.sizes), "read_s": [0.0] * threads,
                      "copy_enqueue_s": [0.0] * threads, "pin_alloc_s": 0.0}
        self.started = False
        self.t0 = self.t_done = 0.0
        self.workers = [threading.Thread(target=self._run, args=(w,), daemon=True) for w in range(threads)]
        if start:
            self.start()

    def preallocate(self) -> None:
        """Every worker's pinned buffers now (e.g. before a clock) instead of in the workers."""
        t0 = time.time()
        for w in range(self.nworkers):
            if self.buffers[w] is None:
                self.buffers[w] = [torch.empty(self.chunk_tokens, dtype=torch.int16, pin_memory=True) for _ in range(2)]
        self.stats["pin_alloc_s"] = max(self.stats["pin_alloc_s"], time.time() - t0)

    def start(self, stream_priority: int = 0) -> None:
        if stream_priority != 0:
            raise ValueError("the copy streams keep the default priority on this platform")
        if self.started:
            raise ValueError("the loader has already started")
        self.started = True
        self.t0 = time.time()
        for i, n in enumerate(self.sizes):
            for a in range(0, max(n, 1), self.chunk_tokens):
                self.work.put((i, a, min(n, a + self.chunk_tokens)))
        for _ in self.workers:
            self.work.put(None)
        for t in self.workers:
            t.start()

    def _run(self, w: int) -> None:
        try:
            if self.cpus:
                os.sched_setaffinity(0, self.cpus)  # this thread
            torch.cuda.set_device(self.device)
            stream = torch.cuda.Stream()
            stream.wait_event(self.filled)
            if self.buffers[w] is None:
                t0 = time.time()
                self.buffers[w] = [torch.empty(self.chunk_tokens, dtype=torch.int16, pin_memory=True) for _ in range(2)]
                with self.lock:
                    self.stats["pin_alloc_s"] = max(self.stats["pin_alloc_s"], time.time() - t0)
            bufs = self.buffers[w]
            views = [memoryview(b.numpy()).cast("B") for b in bufs]
            last = [None, None]  # each buffer's latest copy
            use = 0
            while (item := self.work.get()) is not None:
                i, a, b = item
                if last[use] is not None:
                    last[use].synchronize()
                n = b - a
                t0 = time.time()
                if n:
                    fd = os.open(self.paths[i], os.O_RDONLY)
                    try:
                        got = os.preadv(fd, [views[use][: 2 * n]], HEADER_BYTES + 2 * a)
                    finally:
                        os.close(fd)
                    if got != 2 * n:
                        raise OSError(f"{self.paths[i]}: read {got} of {2 * n} bytes at token {a}")
                t1 = time.time()
                ev = torch.cuda.Event()
                with torch.cuda.stream(stream):
                    if n:
                        at = self.starts[i] + a
                        self.tok[at : at + n].copy_(bufs[use][:n], non_blocking=True)
                    ev.record(stream)
                last[use] = ev
                use ^= 1
                self.stats["read_s"][w] += t1 - t0
                self.stats["copy_enqueue_s"][w] += time.time() - t1
                with self.lock:
                    self.chunk_events[i].append(ev)
                    self.left[i] -= 1
                    done = self.left[i] == 0
                if done:  # the shard's other chunks were enqueued (their events recorded) before this one counted
                    for other in self.chunk_events[i]:
                        stream.wait_event(other)
                    shard_ev = torch.cuda.Event()
                    shard_ev.record(stream)
                    self.events[i] = shard_ev
                    self.chunk_events[i] = []
                    self.ready[i].set()
            stream.synchronize()
            with self.lock:
                self.t_done = max(self.t_done, time.time())
        except BaseException as e:  # noqa: BLE001 - raised to the consumer by wait() / join()
            self.errors.append(e)
            for r in self.ready:
                r.set()

    def wait(self, i: int):
        """Shard i's copy event, once its last chunk is enqueued; raises a worker's error."""
        if not self.started:
            raise ValueError("the loader has not started")
        self.ready[i].wait()
        if self.errors:
            raise self.errors[0]
        return self.events[i]

    def shard_events(self) -> "ShardEvents":
        """Shard i's event on demand (waiting only for shard i): what a build's first scans take as `ready`."""
        return ShardEvents(self)

    def wait_all(self, stream: torch.cuda.Stream | None = None) -> None:
        """The consumer's stream (the current one by default) waits for every shard's copies."""
        s = stream or torch.cuda.current_stream()
        for i in range(len(self.paths)):
            s.wait_event(self.wait(i))

    def join(self) -> None:
        """Every worker done and every copy complete; stats["seconds"] from start to the last copy."""
        for t in self.workers:
            t.join()
        if self.errors:
            raise self.errors[0]
        torch.cuda.synchronize()
        self.stats["seconds"] = self.t_done - self.t0

    def release(self) -> None:
        """The pinned staging buffers freed (after the clock)."""
        if self.started:
            self.join()
        self.buffers = [None] * self.nworkers


class ShardEvents:
    """A loader's per-shard events as a sequence: indexing waits for that shard's last chunk to be enqueued."""

    def __init__(self, loader: Loader):
        self.loader = loader

    def __len__(self) -> int:
        return len(self.loader.paths)

    def __getitem__(self, i: int):
        return self.loader.wait(i)
