"""Build of the HIP libraries (gfx950) in-tree: the csrc/ sources compiled with hipcc and linked into
ngram_amd/_lib/libngram_amd.so (the gpu_val_stats flavour of the C ABI plus the engine's own entry points) and
ngram_amd/_lib/libngram_amd_record.so (the record flavour: the same names with the record's signatures). As the
reference builds its kernels once per source digest into a cache directory under a file lock
(old_records/gpu_val_stats.py:102-130, record_367_gpu_counts/track_1_short/counts/build.py:58-71), a build here:
  * holds an exclusive lock on _lib/.build.lock for its whole length (concurrent builds take turns);
  * compiles into a private object directory of its own (_lib/obj.<pid>.<random>), removed afterwards;
  * links each library to a temporary name and renames it into place (a reader never sees half a library);
  * writes _lib/BUILD_DIGEST: the SHA-256 of every source and header, the flags and the compiler, so `build(force=
    False)` (and `stale()`) know whether the libraries in place were built from the sources in the tree.
hipcc --offload-arch=gfx950 -O3."""

from __future__ import annotations

import fcntl
import hashlib
import json
import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = ROOT / "csrc"
OUT_DIR = PKG / "_lib"
LIB_NAME = "libngram_amd.so"
RECORD_LIB_NAME = "libngram_amd_record.so"
DIGEST_FILE = OUT_DIR / "BUILD_DIGEST"
LOCK_FILE = OUT_DIR / ".build.lock"
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


def digest(extra: list[str] | None = None) -> str:
    """SHA-256 over every source and header under csrc/ (paths and contents), the flags and the compiler path."""
    h = hashlib.sha256()
    for p in sorted(CSRC.rglob("*")):
        if p.is_file() and p.suffix in (".hip", ".h", ".hpp", ".cpp"):
            h.update(str(p.relative_to(CSRC)).encode())
            h.update(b"\0")
            h.update(p.read_bytes())
            h.update(b"\0")
    h.update(json.dumps([HIPCC, FLAGS, extra or [], LIBS]).encode())
    return h.hexdigest()


def stale(extra: list[str] | None = None) -> bool:
    """Whether the libraries in place are missing or were built from other sources (or flags) than the tree's."""
    if not all(lib_path(n).exists() for n in LIBS) or not DIGEST_FILE.exists():
        return True
    try:
        return json.loads(DIGEST_FILE.read_text()).get("digest") != digest(extra)
    except (ValueError, OSError):
        return True


def build(verbose: bool = False, extra: list[str] | None = None, force: bool = True) -> Path:
    """Compile every source (in parallel) and link the libraries, under the build lock; returns the main library's
    path. force=False: nothing is done when the libraries in place match the tree's digest. Raises on a compiler
    error (the libraries in place are then left as they were)."""
    OUT_DIR.mkdir(parents=True, exist_ok=True)
    extra = extra or []
    with open(LOCK_FILE, "a+") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        try:
            want = digest(extra)
            if not force and not stale(extra):
                return lib_path()
            obj_dir = Path(tempfile.mkdtemp(prefix=f"obj.{os.getpid()}.", dir=OUT_DIR))
            try:
                _compile_and_link(obj_dir, extra, verbose)
            finally:
                shutil.rmtree(obj_dir, ignore_errors=True)
            tmp = DIGEST_FILE.with_suffix(f".tmp{os.getpid()}")
            tmp.write_text(json.dumps({"digest": want, "arch": ARCH, "libraries": sorted(LIBS)}) + "\n")
            tmp.replace(DIGEST_FILE)
        finally:
            fcntl.flock(lock, fcntl.LOCK_UN)
    return lib_path()


def _compile_and_link(obj_dir: Path, extra: list[str], verbose: bool) -> None:
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
            tmp.unlink(missing_ok=True)
            raise RuntimeError(f"link of {name} failed:\n{r.stderr}")
        tmp.replace(out)


if __name__ == "__main__":
    force = "--if-stale" not in sys.argv
    print(build(verbose=True, force=force))
