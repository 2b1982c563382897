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
        self._fns: dict = {}

    def _fn(self, name: str):
        fn = self._fns.get(name)
        if fn is None:
            fn = self.so[name]  # a function object of its own (size() sets another return type on the shared one)
            fn.restype = ctypes.c_int
            self._fns[name] = fn
        return fn

    def __call__(self, name: str, *args) -> int:
        # the host side of every launch: kept short, since a build issues a few hundred of them back to back
        conv = []
        for a in args:
            if isinstance(a, torch.Tensor):
                conv.append(ctypes.c_void_p(a.data_ptr()))
            elif a is None:
                conv.append(None)
            elif isinstance(a, int):
                conv.append(ctypes.c_int64(a))
            elif isinstance(a, (ctypes._SimpleCData, ctypes.Array)):
                conv.append(a)
            else:
                raise TypeError(f"{name}: argument {a!r}")
        conv.append(ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(torch._C._cuda_getDevice())))
        rc = self._fn(name)(*conv)
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

    def fill(self, t: torch.Tensor, v: int) -> torch.Tensor:
        """Every element of the contiguous device tensor t set to v, 0 or -1 (a byte pattern: all zeros or all ones),
        by this library's fill kernel on the current stream; returns t."""
        if v not in (0, -1) or not t.is_contiguous():
            raise ValueError("fill takes 0 or -1 over a contiguous tensor")
        nbytes = t.numel() * t.element_size()
        if nbytes % 8 == 0:
            self("ng_fill_u64", t, nbytes // 8, ctypes.c_uint64(0 if v == 0 else (1 << 64) - 1))
        elif nbytes % 4 == 0:
            self("ng_fill_u32", t, nbytes // 4, ctypes.c_uint32(0 if v == 0 else (1 << 32) - 1))
        else:
            t.fill_(v)
        return t

    def zeros(self, shape, dtype, device) -> torch.Tensor:
        """torch.zeros without a framework kernel (this library's fill)."""
        return self.fill(torch.empty(shape, dtype=dtype, device=device), 0)

    def full_ones(self, shape, dtype, device) -> torch.Tensor:
        """A tensor of -1 (every bit set) without a framework kernel."""
        return self.fill(torch.empty(shape, dtype=dtype, device=device), -1)

    def plain(self, name: str, *args) -> int:
        """A call without the stream argument (e.g. max_pbits)."""
        return self._fn(name)(*args)

    def size(self, name: str, *args: int) -> int:
        """A sizing call without the stream argument that returns int64 (its arguments int64)."""
        fn = getattr(self.so, name)
        fn.restype = ctypes.c_int64
        return int(fn(*(ctypes.c_int64(a) for a in args)))
