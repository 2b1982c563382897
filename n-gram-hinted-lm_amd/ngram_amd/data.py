"""Token streams: the reference's shard file format, and the seeded synthetic streams the benchmark configurations use.

Shard file (reference `exact_match/src/lib.rs:23-25,46-56`, `old_records/gpu_val_stats.py:194-198`): 256 little-endian
int32 (magic 20240520, version 1, token count, then zeros) = 1024 bytes, then the tokens as little-endian uint16.

Synthetic stream (one per (config, stream name)): documents of a geometric body length (mean 1024, at least 1) each
followed by the end-of-text token BOS = 50256; body tokens drawn from a Zipf(s) law over ranks 1..50256, rank r mapped to
token id perm[r - 1] by a fixed seeded permutation of 0..50255 (BOS is never drawn); a share of the documents then has a
window overwritten by a copy of a span of an earlier document (of the same stream, before any copy was applied) or of a
source stream (the training corpus, for held-out query streams).

Every body token is a pure function of (stream key, absolute position): a counter-based draw (SplitMix64's finalizer
over key + (position + 1) * 2^64/phi, Steele, Lea & Flood 2014), a 53-bit uniform, and the first Zipf CDF entry above
it. The plan (document lengths, copies) is drawn on the host with numpy's PCG64. So the GPU generator
(`gen_tokens`, `gen_set`, `gen_copies` in the HIP library) and this module's numpy generator produce the same bytes."""

from __future__ import annotations

import hashlib
import os
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

HEADER_BYTES = 1024
HEADER_INTS = HEADER_BYTES // 4
MAGIC = 20240520
VERSION = 1
BOS = 50256
VOCAB = 50257
SHARD_TOKENS = 100_000_000  # tokens per FineWeb training shard (src/retrieval_blog_post/kgram.py:23)
GOLDEN = 0x9E3779B97F4A7C15
M64 = (1 << 64) - 1


# ---------------------------------------------------------------------------------------------------------------
# Shard files
# ---------------------------------------------------------------------------------------------------------------

def write_shard(path: str | os.PathLike, tokens: np.ndarray) -> None:
    """Write `tokens` (uint16) as a shard file."""
    tokens = np.ascontiguousarray(tokens, dtype="<u2")
    header = np.zeros(HEADER_INTS, dtype="<i4")
    header[0], header[1], header[2] = MAGIC, VERSION, len(tokens)
    with open(path, "wb") as f:
        f.write(header.tobytes())
        f.write(tokens.tobytes())


def shard_tokens(path: str | os.PathLike) -> int:
    """The token count of a shard file; ValueError on a bad header or a size that does not match it (the reference's
    `open_shard`, exact_match/src/lib.rs:46-56)."""
    header = np.fromfile(path, dtype="<i4", count=HEADER_INTS)
    if len(header) < 3 or header[0] != MAGIC or header[1] != VERSION or header[2] < 0:
        raise ValueError(f"invalid shard {path}")
    n = int(header[2])
    if Path(path).stat().st_size != HEADER_BYTES + 2 * n:
        raise ValueError(f"invalid shard {path}")
    return n


def read_shard(path: str | os.PathLike) -> np.ndarray:
    """The tokens of a shard file (uint16, memory-mapped read-only)."""
    n = shard_tokens(path)
    return np.memmap(path, dtype="<u2", mode="r", offset=HEADER_BYTES, shape=(n,))


GAP = 32  # SENT tokens at least before every shard (and after the last) in a device buffer: >= any short context


def pack_layout(sizes: list[int], gap: int = GAP) -> tuple[list[int], int]:
    """Where shards of `sizes` tokens go in one device buffer: each shard starts on a multiple of 32 (a bitmap word)
    with at least `gap` SENT tokens before it, and the buffer ends with at least `gap` SENT tokens, its length a
    multiple of 32. So a context reaching back past its shard's start holds a SENT (and matches no query context), a
    position whose next token is SENT is not an occurrence, and the scans' bitmaps cover the buffer in whole words.
    Returns (starts, length)."""
    starts, end = [], 0
    for n in sizes:
        at = -(-(end + gap) // 32) * 32
        starts.append(at)
        end = at + int(n)
    return starts, -(-(end + gap) // 32) * 32


def device_tokens(shards: list, device="cuda"):
    """Shards (uint16 arrays, or shard file paths) copied into one int16 device buffer laid out by pack_layout:
    (tok, sizes, starts, length). Synchronous: ngram_amd.loader overlaps the reads and copies with other work."""
    import torch

    arrays = [read_shard(s) if isinstance(s, (str, os.PathLike)) else np.asarray(s, np.uint16) for s in shards]
    sizes = [len(a) for a in arrays]
    starts, length = pack_layout(sizes)
    tok = torch.full((length,), -1, dtype=torch.int16, device=device)
    for a, at in zip(arrays, starts):
        if len(a):
            tok[at : at + len(a)].copy_(torch.from_numpy(np.ascontiguousarray(a).view(np.int16)))
    return tok, sizes, starts, length


def segments(x: np.ndarray, breaks: list[int] | tuple[int, ...] = ()) -> np.ndarray:
    """Per position of `x`, the tokens of its segment up to and including it (int32): a segment starts at position 0,
    at every BOS and at every position of `breaks`. A position's k-context is valid iff this is >= k (reference
    `exact_match/src/kgram.rs:224-234`, `old_records/gpu_val_stats.py:789-792`, `counts/build.py:144-158`)."""
    n = len(x)
    start = np.asarray(x) == BOS
    if n:
        start[0] = True
    for b in breaks:
        start[b] = True
    idx = np.arange(n, dtype=np.int64)
    seg = np.maximum.accumulate(np.where(start, idx, 0)) if n else idx
    return (idx - seg + 1).astype(np.int32)


# ---------------------------------------------------------------------------------------------------------------
# Counter-based draws
# ---------------------------------------------------------------------------------------------------------------

def mix64(h: np.ndarray) -> np.ndarray:
    """SplitMix64's finalizer on uint64 arrays (a bijection)."""
    h = h.astype(np.uint64, copy=True)
    h ^= h >> np.uint64(30)
    h *= np.uint64(0xBF58476D1CE4E5B9)
    h ^= h >> np.uint64(27)
    h *= np.uint64(0x94D049BB133111EB)
    h ^= h >> np.uint64(31)
    return h


def stream_key(*parts) -> int:
    """A 64-bit key for a named stream (deterministic across processes and machines)."""
    digest = hashlib.blake2b(repr(parts).encode(), digest_size=8).digest()
    return int.from_bytes(digest, "little")


def uniforms(key: int, start: int, n: int) -> np.ndarray:
    """The 53-bit uniforms in [0, 1) of positions [start, start + n) of stream `key`."""
    idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        h = mix64(np.uint64(key) + idx * np.uint64(GOLDEN))
    return (h >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


@dataclass(frozen=True)
class Zipf:
    """Zipf(s) over ranks 1..50256 and the rank -> token id permutation of one configuration."""

    s: float
    seed: int
    cdf: np.ndarray = field(repr=False)  # float64 [50256], cdf[-1] == 1
    perm: np.ndarray = field(repr=False)  # uint16 [50256]

    @staticmethod
    def make(s: float = 1.1, seed: int = 0) -> "Zipf":
        w = np.arange(1, BOS + 1, dtype=np.float64) ** -s
        cdf = np.cumsum(w) / w.sum()
        cdf[-1] = 1.0
        perm = np.random.Generator(np.random.PCG64(seed)).permutation(BOS).astype(np.uint16)
        return Zipf(s, seed, cdf, perm)

    def tokens(self, key: int, start: int, n: int) -> np.ndarray:
        """The pure Zipf draws of positions [start, start + n) of stream `key` (uint16)."""
        out = np.empty(n, dtype=np.uint16)
        step = 1 << 22
        for a in range(0, n, step):
            b = min(n, a + step)
            r = np.searchsorted(self.cdf, uniforms(key, start + a, b - a), side="right")
            np.minimum(r, BOS - 1, out=r)
            out[a:b] = self.perm[r]
        return out


# ---------------------------------------------------------------------------------------------------------------
# Stream plans
# ---------------------------------------------------------------------------------------------------------------

@dataclass
class Plan:
    """A stream's layout: n tokens, the positions of its BOS tokens (each ends a document), and its copies
    (dst, src, length) applied to the pure draws: src indexes this stream's pure draws (`external` False) or the source
    stream (`external` True)."""

    key: int
    n: int
    eos: np.ndarray  # int64 positions
    doc_start: np.ndarray  # int64, first body token of each document
    doc_len: np.ndarray  # int64, body lengths (without the BOS)
    copies: np.ndarray  # int64 [m, 3]: dst, src, length
    external: bool


def make_plan(key: int, n: int, *, mean_doc: int = 1024, copy_rate=0.0, copy_len=(32, 256),
              source: "Plan | None" = None, seed_extra: int = 0) -> Plan:
    """The plan of an n-token stream. `copy_rate` is a share of documents, or a callable of the document's start
    position / n (a ramp). With `source`, copies come from that stream's documents, else from earlier documents of this
    one."""
    rng = np.random.Generator(np.random.PCG64(key ^ seed_extra))
    p = 1.0 / mean_doc
    lens = []
    total = 0
    while total < n:
        m = max(16, int((n - total) / (mean_doc + 1) * 1.1) + 16)
        body = rng.geometric(p, size=m).astype(np.int64)
        lens.append(body)
        total += int((body + 1).sum())
    body = np.concatenate(lens)
    ends = np.cumsum(body + 1)  # one past each document's BOS
    d = int(np.searchsorted(ends, n, side="left")) + 1  # documents touching [0, n)
    body = body[:d]
    ends = ends[:d]
    doc_start = ends - body - 1
    eos = ends - 1
    eos = eos[eos < n]
    body = np.minimum(body, n - doc_start)  # the last document may be cut
    copies = []
    lo, hi = copy_len
    rate = copy_rate
    src_start = source.doc_start if source is not None else doc_start
    src_len = source.doc_len if source is not None else body
    for j in range(d):
        r = rate(doc_start[j] / n) if callable(rate) else rate
        u = rng.random()
        if r <= 0 or u >= r or body[j] < 2:
            continue
        if source is None:
            if j == 0:
                continue
            s = int(rng.integers(0, j))
        else:
            s = int(rng.integers(0, len(src_start)))
        length = int(rng.integers(lo, hi + 1))
        length = min(length, int(body[j]), int(src_len[s]))
        if length < 1:
            continue
        dst = int(doc_start[j] + rng.integers(0, body[j] - length + 1))
        src = int(src_start[s] + rng.integers(0, src_len[s] - length + 1))
        copies.append((dst, src, length))
    cp = np.array(copies, dtype=np.int64).reshape(-1, 3)
    return Plan(key, n, eos.astype(np.int64), doc_start.astype(np.int64), body.astype(np.int64), cp, source is not None)


def realize(plan: Plan, zipf: Zipf, source_tokens: np.ndarray | None = None) -> np.ndarray:
    """The stream's tokens (uint16) on the host: pure draws, BOS at document ends, then the copies."""
    pure = zipf.tokens(plan.key, 0, plan.n)
    pure[plan.eos] = BOS
    if len(plan.copies) == 0:
        return pure
    out = pure.copy()
    src = source_tokens if plan.external else pure
    for dst, s, length in plan.copies:
        out[dst : dst + length] = src[s : s + length]
    return out


def realize_gpu(plan: Plan, zipf: Zipf, lib, source=None, out=None):
    """The stream's tokens generated on the GPU by the library's gen_tokens / gen_set / gen_copies (the same bytes as
    `realize`): a torch int16 tensor (uint16 bits) of plan.n tokens, or written into `out`. `source`: the source
    stream's tokens on the GPU (int16 tensor), needed when the plan's copies are external."""
    import torch

    from .lib import i32, u64

    if plan.external and source is None:
        raise ValueError("the plan copies from a source stream: pass its tokens")
    dev = torch.device("cuda", torch.cuda.current_device())
    if out is None:
        out = torch.empty(plan.n, dtype=torch.int16, device=dev)
    elif out.numel() != plan.n or out.dtype != torch.int16:
        raise ValueError("out must be int16 of plan.n tokens")
    cdf = torch.from_numpy(zipf.cdf).to(dev)
    perm = torch.from_numpy(zipf.perm.view(np.int16)).to(dev)
    lib("gen_tokens", out, 0, plan.n, u64(plan.key), cdf, i32(len(zipf.cdf)), perm)
    eos = torch.from_numpy(plan.eos).to(dev)
    lib("gen_set", out, eos, len(plan.eos), i32(BOS))
    if len(plan.copies):
        cp = torch.from_numpy(np.ascontiguousarray(plan.copies)).to(dev)
        lib("gen_copies", out, cp, len(plan.copies), source if plan.external else None, u64(plan.key), cdf,
            i32(len(zipf.cdf)), perm)
    torch.cuda.current_stream().synchronize()
    return out


# ---------------------------------------------------------------------------------------------------------------
# The benchmark configurations c1-c5
# ---------------------------------------------------------------------------------------------------------------

@dataclass(frozen=True)
class Config:
    name: str
    train_tokens: int
    query_tokens: int  # query stream length (inputs + 1)
    levels: tuple[int, ...]
    topk: int
    copy_rate: float
    copy_len: tuple[int, int]
    query_copy_rate: float
    query_copy_len: tuple[int, int]
    match_cap: int = 0
    shard_tokens: int = SHARD_TOKENS


CONFIGS = {
    "c1": Config("c1", 4 << 20, (256 << 10) + 1, (2, 3), 1, 0.10, (32, 256), 0.10, (32, 256), match_cap=32,
                 shard_tokens=1 << 20),
    "c2": Config("c2", 100_000_000, 8_000_000 + 1, (2, 3, 4), 4, 0.10, (32, 256), 0.10, (32, 256)),
    "c3": Config("c3", 1_000_000_000, 16_000_000 + 1, (2, 3, 4, 5, 6, 7, 8), 4, 0.05, (32, 1024), 0.05, (32, 1024)),
    "c5": Config("c5", 1_000_000_000, 64_000_000 + 1, (), 1, 0.05, (32, 1024), 0.15, (16, 2048), match_cap=64),
}


@dataclass
class Corpus:
    """A configuration's streams on the host: the training shards and the query stream (inputs + one more token)."""

    config: Config
    zipf: Zipf
    train_plan: Plan
    query_plan: Plan
    train: np.ndarray  # the concatenated training tokens
    bounds: np.ndarray  # shard starts in `train`, then its length
    query: np.ndarray

    def shards(self) -> list[np.ndarray]:
        return [self.train[a:b] for a, b in zip(self.bounds[:-1], self.bounds[1:])]

    def write(self, directory: str | os.PathLike) -> tuple[list[str], str]:
        """The shards and the query stream as shard files in `directory`: (train paths, query path)."""
        d = Path(directory)
        d.mkdir(parents=True, exist_ok=True)
        paths = []
        for i, s in enumerate(self.shards()):
            p = d / f"train_{i:06d}.bin"
            write_shard(p, s)
            paths.append(str(p))
        q = d / "val_000000.bin"
        write_shard(q, self.query)
        return paths, str(q)


def train_bounds(n: int, shard: int) -> np.ndarray:
    return np.array(list(range(0, n, shard)) + [n], dtype=np.int64)


def make_plans(cfg: Config, train_tokens: int | None = None, query_tokens: int | None = None) -> tuple[Zipf, Plan, Plan]:
    """The Zipf law and the train / query plans of configuration `cfg` (token counts overridable, for scaled-down
    tests; the streams are then prefixes of nothing: a different count gives a different plan)."""
    t = train_tokens or cfg.train_tokens
    q = query_tokens or cfg.query_tokens
    zipf = Zipf.make(1.1, seed=stream_key(cfg.name, "perm") & 0xFFFFFFFF)
    tp = make_plan(stream_key(cfg.name, "train", t), t, copy_rate=cfg.copy_rate, copy_len=cfg.copy_len)
    qp = make_plan(stream_key(cfg.name, "query", q), q, copy_rate=cfg.query_copy_rate, copy_len=cfg.query_copy_len,
                   source=tp)
    return zipf, tp, qp


def make_corpus(name: str, train_tokens: int | None = None, query_tokens: int | None = None,
                shard_tokens: int | None = None) -> Corpus:
    """Configuration `name`'s streams on the host (numpy)."""
    cfg = CONFIGS[name]
    zipf, tp, qp = make_plans(cfg, train_tokens, query_tokens)
    train = realize(tp, zipf)
    query = realize(qp, zipf, train)
    bounds = train_bounds(tp.n, shard_tokens or cfg.shard_tokens)
    return Corpus(cfg, zipf, tp, qp, train, bounds, query)


@dataclass
class DeviceCorpus:
    """A configuration's streams generated on the GPU: the training tokens without gaps (`flat`, int16), their shard
    bounds, the same tokens laid out for the scans (`tok`, data.pack_layout's `sizes` / `starts`) and the query stream
    (`query`, int16: the inputs, then the last target)."""

    config: Config
    zipf: Zipf
    train_plan: Plan
    flat: object
    bounds: np.ndarray
    tok: object
    sizes: list
    starts: list
    query: object


def device_corpus(name: str, train_tokens: int | None = None, query_tokens: int | None = None, lib=None,
                  shard_tokens: int | None = None) -> DeviceCorpus:
    """Configuration `name`'s streams generated on the GPU (byte-identical to make_corpus's)."""
    import torch

    from .lib import Lib

    cfg = CONFIGS[name]
    zipf, tp, qp = make_plans(cfg, train_tokens, query_tokens)
    lib = lib or Lib()
    flat = realize_gpu(tp, zipf, lib)
    q = realize_gpu(qp, zipf, lib, source=flat)
    bounds = train_bounds(tp.n, shard_tokens or cfg.shard_tokens)
    sizes = [int(b - a) for a, b in zip(bounds[:-1], bounds[1:])]
    starts, length = pack_layout(sizes)
    tok = torch.full((length,), -1, dtype=torch.int16, device=flat.device)
    for a, b, at in zip(bounds[:-1], bounds[1:], starts):
        tok[at : at + (b - a)].copy_(flat[a:b])
    return DeviceCorpus(cfg, zipf, tp, flat, bounds, tok, sizes, starts, q)


C4_STEPS = 92
C4_STEP_TOKENS = 1 << 19


def c4_stream(steps: int = C4_STEPS, step_tokens: int = C4_STEP_TOKENS, copy_rate_end: float = 0.20):
    """Configuration c4: a stream of `steps` x `step_tokens` tokens (same generator: Zipf(1.1)
    documents ending with BOS), the share of documents with a copied span (32-256 tokens of an earlier document)
    ramping linearly from 0 at the stream's start to `copy_rate_end` at its end. Returns (zipf, plan, spans), spans
    (s * step_tokens, (s + 1) * step_tokens, s): step s trains its inputs and, as its last target, the next step's
    first token."""
    n = steps * step_tokens
    zipf = Zipf.make(1.1, seed=stream_key("c4", "perm") & 0xFFFFFFFF)
    plan = make_plan(stream_key("c4", "stream", n), n, copy_rate=lambda f: copy_rate_end * f, copy_len=(32, 256))
    spans = np.array([(s * step_tokens, (s + 1) * step_tokens, s) for s in range(steps)], np.int64)
    return zipf, plan, spans
