"""CPU: the C-ABI libraries build for gfx950, load, and export every entry point include/*.h declares (no GPU calls)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
# header -> the library that exports its declarations
HEADERS = {"ngram_amd.h": "libngram_amd.so", "ngram_amd_record.h": "libngram_amd_record.so"}


def declared_symbols(header: str) -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / header).read_text(), flags=re.S)
    return re.findall(r"^\s*(?:int|size_t|void|ng_i64|ng_u64)\s+(\w+)\s*\(", text, flags=re.M)


@pytest.fixture(scope="module")
def libs():
    from ngram_amd import build

    if not all(build.lib_path(n).exists() for n in HEADERS.values()):
        build.build()
    return {h: ctypes.CDLL(str(build.lib_path(n))) for h, n in HEADERS.items()}


def test_every_header_is_mapped():
    assert sorted(p.name for p in (ROOT / "include").glob("*.h")) == sorted(HEADERS)


def test_header_declares_the_reference_abi():
    gvs = set(declared_symbols("ngram_amd.h"))
    reference = {"val_keys", "val_verify", "val_homes", "scan_level", "subpart_count", "subpart_scatter", "aggregate",
                 "max_pbits", "popcount", "part_count", "part_scatter", "sort_pairs", "inclusive_max",
                 "reduce_by_key", "seg_bounds", "ctx_tot", "rank_keys", "rank_scatter", "pos_outputs",
                 "variant_rows"}
    assert reference <= gvs, reference - gvs
    record = set(declared_symbols("ngram_amd_record.h"))
    reference_rec = {"val_keys", "val_verify", "val_homes", "scan_level", "part_count", "part_scatter", "sort_pairs",
                     "inclusive_max", "reduce_by_key", "seg_bounds", "ctx_tot", "rank_keys", "rank_scatter",
                     "pos_outputs"}
    assert reference_rec <= record, reference_rec - record


def test_libraries_export_every_declared_symbol(libs):
    for h, so in libs.items():
        missing = [n for n in declared_symbols(h) if not hasattr(so, n)]
        assert not missing, (h, missing)


def test_product_does_not_import_the_oracle():
    pkg = ROOT / "n-gram-hinted-lm_amd"
    for f in list(pkg.rglob("*.py")) + list(pkg.rglob("*.hip")) + list(pkg.rglob("*.h")):
        text = f.read_text()
        assert "import oracle" not in text and "liboracle" not in text, f


def test_build_digest_tracks_the_sources(tmp_path, monkeypatch):
    """build.digest() covers every source and header under csrc/ and the flags: a changed source, a new header or
    another flag gives another digest (stale() then tells that the libraries in place are not the tree's)."""
    from ngram_amd import build

    src = tmp_path / "csrc"
    (src / "abi").mkdir(parents=True)
    (src / "a.hip").write_text("int a;\n")
    (src / "abi" / "b.h").write_text("int b;\n")
    monkeypatch.setattr(build, "CSRC", src)
    d0 = build.digest()
    assert d0 == build.digest()
    (src / "a.hip").write_text("int a2;\n")
    d1 = build.digest()
    (src / "abi" / "c.h").write_text("\n")
    d2 = build.digest()
    assert len({d0, d1, d2, build.digest(["-DX"])}) == 4


def test_builds_take_turns_on_the_lock(tmp_path, monkeypatch):
    """A build waits for the lock another holds: a second process's build (here one with nothing to do) returns only
    after the lock is released."""
    import fcntl
    import subprocess
    import sys
    import time

    from ngram_amd import build

    if build.stale():
        pytest.skip("the libraries in place are not the tree's: build() first")
    build.OUT_DIR.mkdir(parents=True, exist_ok=True)
    code = ("import sys, time; sys.path.insert(0, %r); from ngram_amd import build; t = time.time(); "
            "build.build(force=False); print(time.time() - t)") % str(ROOT / "n-gram-hinted-lm_amd")
    with open(build.LOCK_FILE, "a+") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        p = subprocess.Popen([sys.executable, "-c", code], stdout=subprocess.PIPE, text=True)
        time.sleep(1.5)
        assert p.poll() is None  # still waiting for the lock
        fcntl.flock(lock, fcntl.LOCK_UN)
    out, _ = p.communicate(timeout=60)
    assert p.returncode == 0 and float(out.split()[-1]) >= 1.0


def declared_arity(header: str) -> dict[str, int]:
    """Each declared function's parameter count (the header's prototypes, comments removed)."""
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / header).read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(?:int|size_t|void|ng_i64|ng_u64)\s+(\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.M | re.S):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_engine_calls_match_the_header_arity():
    """Every call of an ng_* entry point through the ctypes wrapper (`lib("ng_x", ...)`, `lib.cub("ng_x", ...)` for
    the two-phase ones, `lib.size("ng_x", ...)` for the sizing ones) passes as many arguments as the prototype has,
    less the stream the wrapper appends (and the temp pair `cub` adds): a missing argument would shift the stream into
    another parameter."""
    import ast

    arity = declared_arity("ngram_amd.h")
    files = list((ROOT / "n-gram-hinted-lm_amd").rglob("*.py")) + [ROOT / "bench.py", ROOT / "__graft_entry__.py"]
    files += list((ROOT / "tests").glob("*.py"))
    checked, bad = 0, []
    for f in files:
        for node in ast.walk(ast.parse(f.read_text())):
            if not (isinstance(node, ast.Call) and node.args and isinstance(node.args[0], ast.Constant)):
                continue
            name = node.args[0].value
            if not (isinstance(name, str) and name.startswith("ng_") and name in arity):
                continue
            if node.keywords or any(isinstance(a, ast.Starred) for a in node.args):
                continue
            kind = node.func.attr if isinstance(node.func, ast.Attribute) else ""
            if kind == "size":  # sizing calls take no stream
                want = arity[name]
            else:
                want = arity[name] - (3 if kind == "cub" else 1)
            checked += 1
            if len(node.args) - 1 != want:
                bad.append(f"{f.name}:{node.lineno} {name}: {len(node.args) - 1} arguments, the prototype takes {want}")
    assert checked > 50
    assert not bad, bad
