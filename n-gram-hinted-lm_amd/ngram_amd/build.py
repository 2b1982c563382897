"""Build of the HIP libraries (gfx950) in-tree: the csrc/ sources compiled with hipcc and linked into
ngram_amd/_lib/libngram_amd.so (the gpu_val_stats flavour of the C ABI plus the engine's own entry points) and
ngram_amd/_lib/libngram_amd_record.so (the record flavour: the same names with the record's signatures). The reference
builds its kernels with nvcc into a .so per source digest (old_records/gpu_val_stats.py:102-130,
record_367_gpu_counts/track_1_short/counts/build.py:58-71); here hipcc --offload-arch=gfx950."""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = ROOT / "csrc"
OUT_DIR = PKG / "_lib"
LIB_NAME = "libngram_amd.so"
RECORD_LIB_NAME = "libngram_amd_record.so"
# each library's sources (relative to csrc/); an object shared by both is compiled once
LIBS = {
    LIB_NAME: ["prim.hip", "abi/owner.hip", "abi/gvs.hip", "gen.hip", "engine.hip", "part.hip", "table.hip",
               "online.hip", "rows.hip", "hintrows.hip", "pairs32.hip"],
    RECORD_LIB_NAME: ["prim.hip", "abi/owner.hip", "abi/record.hip"],
}
ARCH = os.environ.get("NGRAM_AMD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
         # compiler-formed packed fp32 ops are kept off (they have given wrong results on these machines)
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def lib_path(name: str = LIB_NAME) -> Path:
    return OUT_DIR / name


def sources() -> list[Path]:
    return sorted({CSRC / s for srcs in LIBS.values() for s in srcs})


def build(verbose: bool = False, extra: list[str] | None = None) -> Path:
    """Compile every source (in parallel) and link the library; returns its path. Raises on a compiler error."""
    OUT_DIR.mkdir(parents=True, exist_ok=True)
    obj_dir = OUT_DIR / "obj"
    obj_dir.mkdir(exist_ok=True)
    extra = extra or []

    def compile_one(src: Path) -> Path:
        obj = obj_dir / (str(src.relative_to(CSRC).with_suffix("")).replace("/", "_") + ".o")
        cmd = [HIPCC, *FLAGS, *extra, "-I", str(CSRC), "-c", str(src), "-o", str(obj)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr}")
        if verbose and r.stderr.strip():
            print(r.stderr, file=sys.stderr)
        return obj

    srcs = sources()
    with ThreadPoolExecutor(max(1, min(len(srcs), os.cpu_count() or 4))) as ex:
        objs = dict(zip(srcs, ex.map(compile_one, srcs)))
    for name, lib_srcs in LIBS.items():
        out = lib_path(name)
        tmp = out.with_suffix(f".so.tmp{os.getpid()}")
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
               *[str(objs[CSRC / s]) for s in lib_srcs]]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link of {name} failed:\n{r.stderr}")
        tmp.replace(out)
    return lib_path()


if __name__ == "__main__":
    print(build(verbose=True))
