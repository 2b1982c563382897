"""The shard loader of the validation statistics' host (the mirror of old_records/gpu_val_stats.py `Loader`
:226-359, `numa_cpus` :199-216): a rank's shard files into one GPU token buffer laid out with SENT gaps, in background
threads, so the copies overlap the query index and the first shards' scans.

Each thread takes every `threads`-th shard, reads it in chunks of `chunk_tokens` with `preadv` (the GIL is released
during the read) into one of two pinned staging buffers of its own, and enqueues the chunk's host-to-device copy on a
HIP stream of its own; a buffer is reused once the copy that last read it has completed (its event), so a thread reads
chunk j + 1 while chunk j crosses PCIe. After a shard's last chunk the thread records the shard's event and sets
`ready[i]`; `wait(i)` returns that event for the consumer's stream to wait on.

Platform differences, each with its reason: mode "register" (the reference pins each shard's tmpfs mapping in place
with cudaHostRegister and copies from it directly) raises ValueError, since this platform refuses to pin memory that
already exists (hipHostRegister), so "pread" is the only mode; the copy streams keep the default priority (`start`
refuses another), since work on streams of other priorities has hung on this platform. Pinned buffers come from
torch's pinned allocator (hipHostMalloc)."""

from __future__ import annotations

import os
import threading
import time
from pathlib import Path

import torch

from .data import HEADER_BYTES


def numa_cpus(device: int) -> set[int]:
    """The CPUs of the GPU's NUMA node that this process may use (empty if unknown) (:199-216)."""
    try:
        p = torch.cuda.get_device_properties(device)
        bus = f"{p.pci_domain_id:04x}:{p.pci_bus_id:02x}:{p.pci_device_id:02x}.0"
        node = int(Path(f"/sys/bus/pci/devices/{bus}/numa_node").read_text())
        if node < 0:
            return set()
        cpus: set[int] = set()
        for part in Path(f"/sys/devices/system/node/node{node}/cpulist").read_text().strip().split(","):
            a, _, b = part.partition("-")
            cpus.update(range(int(a), int(b or a) + 1))
        return cpus & os.sched_getaffinity(0)
    except Exception:  # noqa: BLE001 - an unknown topology only means no pinning of the threads
        return set()


class Loader:
    """Shards `paths` (sizes[i] tokens each) into `tok` (a new int16 [tok_len] GPU buffer of SENT = -1 unless given)
    at starts[i], in `threads` background threads started at construction unless `start` is False. `chunk_tokens`:
    the pinned staging buffers' size in tokens (two per thread). `numa`: run the threads on the GPU's NUMA node.
    `stats`: per-thread read and enqueue seconds, the pinned allocation's, `bytes`, and (after join) `seconds`."""

    def __init__(self, paths: list, tok_len: int, starts: list[int], sizes: list[int], threads: int,
                 mode: str = "pread", chunk_tokens: int = 8 << 20, numa: bool = False, start: bool = True,
                 tok: torch.Tensor | None = None):
        if mode != "pread":
            raise ValueError(f"load mode {mode!r}: only 'pread' (pinning existing memory in place is refused on this "
                             "platform)")
        if not (len(paths) == len(starts) == len(sizes)):
            raise ValueError("paths, starts and sizes must have one entry per shard")
        if threads < 1 or chunk_tokens < 1:
            raise ValueError(f"threads ({threads}) and chunk_tokens ({chunk_tokens}) must be >= 1")
        for st, n in zip(starts, sizes):
            if st < 0 or st + n > tok_len:
                raise ValueError(f"shard at {st} of {n} tokens exceeds the buffer of {tok_len}")
        self.paths, self.starts, self.sizes, self.mode = [str(p) for p in paths], list(starts), list(sizes), mode
        self.tok = torch.full((tok_len,), -1, dtype=torch.int16, device="cuda") if tok is None else tok
        if self.tok.dtype != torch.int16 or self.tok.numel() < tok_len:
            raise ValueError("tok must be an int16 tensor of at least tok_len tokens")
        self.ready = [threading.Event() for _ in self.paths]
        self.events: list = [None] * len(self.paths)
        self.stats = {"mode": mode, "threads": threads, "read_s": [0.0] * threads, "copy_enqueue_s": [0.0] * threads,
                      "pin_alloc_s": 0.0, "bytes": 2 * sum(self.sizes)}
        self.buffers: list = [None] * threads
        self.errors: list[BaseException] = []
        self.chunk_tokens = chunk_tokens
        self.lock = threading.Lock()
        self.device = torch.cuda.current_device()
        self.cpus = numa_cpus(self.device) if numa else set()
        self.t0 = time.time()
        self.t_done = 0.0
        self.threads = [threading.Thread(target=self._work, args=(t,), daemon=True) for t in range(threads)]
        self.started = False
        if start:
            self.start()

    def preallocate(self) -> None:
        """Every thread's two pinned buffers, now (e.g. before a clock) instead of in the threads (:256-263)."""
        t0 = time.time()
        for t in range(len(self.buffers)):
            if self.buffers[t] is None:
                self.buffers[t] = self._pair()
        self.stats["pin_alloc_s"] = max(self.stats["pin_alloc_s"], time.time() - t0)

    def _pair(self) -> list[torch.Tensor]:
        return [torch.empty(self.chunk_tokens, dtype=torch.int16, pin_memory=True) for _ in range(2)]

    def start(self, stream_priority: int = 0) -> None:
        """Start the load threads (:265-272); their copy streams keep the default priority."""
        if stream_priority != 0:
            raise ValueError("the copy streams keep the default priority on this platform")
        if self.started:
            raise ValueError("the loader has already started")
        self.started = True
        self.t0 = time.time()
        for t in self.threads:
            t.start()

    def _work(self, t: int) -> None:
        try:
            if self.cpus:
                os.sched_setaffinity(0, self.cpus)  # this thread only (Linux)
            torch.cuda.set_device(self.device)
            stream = torch.cuda.Stream()
            if self.buffers[t] is None:
                r0 = time.time()
                self.buffers[t] = self._pair()
                with self.lock:
                    self.stats["pin_alloc_s"] = max(self.stats["pin_alloc_s"], time.time() - r0)
            buffers, used = self.buffers[t], [None, None]
            views = [memoryview(b.numpy()).cast("B") for b in buffers]
            j = 0
            for i in range(t, len(self.paths), len(self.threads)):
                path, n, dst = self.paths[i], self.sizes[i], self.starts[i]
                ev = None
                fd = os.open(path, os.O_RDONLY)
                try:
                    for a in range(0, n, self.chunk_tokens):
                        c = min(n, a + self.chunk_tokens) - a
                        b = j % 2
                        j += 1
                        if used[b] is not None:
                            used[b].synchronize()
                        r0 = time.time()
                        if os.preadv(fd, [views[b][: 2 * c]], HEADER_BYTES + 2 * a) != 2 * c:
                            raise OSError(f"short read of {path}")
                        r1 = time.time()
                        with torch.cuda.stream(stream):
                            self.tok[dst + a : dst + a + c].copy_(buffers[b][:c], non_blocking=True)
                            ev = torch.cuda.Event()
                            ev.record(stream)
                        used[b] = ev
                        self.stats["read_s"][t] += r1 - r0
                        self.stats["copy_enqueue_s"][t] += time.time() - r1
                finally:
                    os.close(fd)
                if ev is None:  # an empty shard: nothing to copy
                    ev = torch.cuda.Event()
                    ev.record(stream)
                self.events[i] = ev
                self.ready[i].set()
            stream.synchronize()
            with self.lock:
                self.t_done = max(self.t_done, time.time())
        except BaseException as e:  # noqa: BLE001 - handed to the consumer by wait()/join()
            self.errors.append(e)
            for r in self.ready:
                r.set()

    def wait(self, i: int):
        """Shard i's copy event, once enqueued (:333-338); raises a load thread's error."""
        if not self.started:
            raise ValueError("the loader has not started")
        self.ready[i].wait()
        if self.errors:
            raise self.errors[0]
        return self.events[i]

    def wait_all(self, stream: torch.cuda.Stream | None = None) -> None:
        """The consumer's stream (the current one by default) waits for every shard's copy."""
        s = torch.cuda.current_stream() if stream is None else stream
        for i in range(len(self.paths)):
            s.wait_event(self.wait(i))

    def join(self) -> None:
        """Every thread done and every copy complete (:340-345); `stats["seconds"]` from start to the last copy."""
        for t in self.threads:
            t.join()
        if self.errors:
            raise self.errors[0]
        torch.cuda.synchronize()
        self.stats["seconds"] = self.t_done - self.t0

    def release(self) -> None:
        """The pinned staging buffers freed (after the clock)."""
        if self.started:
            self.join()
        self.buffers = [None] * len(self.buffers)
