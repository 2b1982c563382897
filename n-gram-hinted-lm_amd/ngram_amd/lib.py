"""The HIP library through ctypes, with the reference's calling convention (old_records/gpu_val_stats.py:133-167,
record_367_gpu_counts/track_1_short/counts/build.py:74-92): tensors as their data pointers, None as NULL, ctypes
scalars as given, Python ints as int64, the current torch stream appended last; a nonzero return raises
RuntimeError(f"{name} returned {rc}"). `cub(name, ...)` runs a two-phase temp-storage call (query, allocate, run).

There is no fallback: a missing library raises (build it first with __graft_entry__.build() or
`python -m ngram_amd.build`)."""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

from .build import lib_path

_loaded: dict[str, ctypes.CDLL] = {}


def load(path: str | Path | None = None) -> ctypes.CDLL:
    p = Path(path) if path is not None else lib_path()
    key = str(p)
    if key not in _loaded:
        if not p.exists():
            raise FileNotFoundError(f"{p}: the HIP library is not built (run __graft_entry__.build())")
        _loaded[key] = ctypes.CDLL(str(p))
    return _loaded[key]


def i32(x: int) -> ctypes.c_int:
    return ctypes.c_int(x)


def u64(x: int) -> ctypes.c_uint64:
    return ctypes.c_uint64(x)


class Lib:
    """The kernels through ctypes: tensors as their data pointers, on the current stream; a nonzero return raises."""

    def __init__(self, path: str | Path | None = None):
        self.so = load(path)

    def __call__(self, name: str, *args) -> int:
        conv = []
        for a in args:
            if isinstance(a, torch.Tensor):
                conv.append(ctypes.c_void_p(a.data_ptr()))
            elif a is None:
                conv.append(ctypes.c_void_p(0))
            elif isinstance(a, (ctypes._SimpleCData, ctypes.Array)):
                conv.append(a)
            elif isinstance(a, int):
                conv.append(ctypes.c_int64(a))
            else:
                raise TypeError(f"{name}: argument {a!r}")
        conv.append(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        fn = getattr(self.so, name)
        fn.restype = ctypes.c_int
        rc = fn(*conv)
        if rc != 0:
            raise RuntimeError(f"{name} returned {rc}")
        return rc

    def cub(self, name: str, *args) -> None:
        """A two-phase temp-storage call: its temp bytes queried, allocated (a torch tensor) and the call run."""
        size = ctypes.c_size_t(0)
        ptr = ctypes.c_void_p(ctypes.addressof(size))
        self(name, None, ptr, *args)
        temp = torch.empty(max(size.value, 1), dtype=torch.uint8, device="cuda")
        self(name, temp, ptr, *args)
        del temp

    def plain(self, name: str, *args) -> int:
        """A call without the stream argument (e.g. max_pbits)."""
        fn = getattr(self.so, name)
        fn.restype = ctypes.c_int
        return fn(*args)

    def size(self, name: str, *args: int) -> int:
        """A sizing call without the stream argument that returns int64 (its arguments int64)."""
        fn = getattr(self.so, name)
        fn.restype = ctypes.c_int64
        return int(fn(*(ctypes.c_int64(a) for a in args)))
