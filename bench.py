"""Benchmark of the n-gram hint path on one MI355X: the one-GPU share of the record's GPU counts build at
configuration c3: a 1B-token seeded synthetic corpus (10 shards of 100M tokens, Zipf(1.1) over permuted ids,
geometric documents of mean 1024 ending with BOS 50256, 5% of documents with a copied span of 32-1024 tokens), exact
counts of the query contexts for n = 2..8, then for 16M query positions each level's tot / dist / cnt, the top-4 next
tokens with counts, and hit/miss. One step = one whole count build + query over the resident corpus and queries.

Prints one JSON line: value = corpus tokens counted per second (T x steps / timed seconds), plus query positions/s;
`roofline`: the dominant kernel (the single launch class that takes the most time per step: a level's scan) at its
algorithmic bytes (2 per corpus position the scan reads -- every position of its range for a dense scan, the listed
positions for a gated one -- plus 8 per hit emitted) over its launch durations (HIP events on its stream); beside it the
same for every level scan together (`roofline_family`), for the count path (scans, partition, LDS counts: 2 per
position read + 16 per hit) and for the whole build (2 T + 16 E over the step); `parity`: the GPU's outputs against
the oracle's on the CPU baseline's sample (every output of the first shard x the first query positions) and on
windows of query positions counted over the whole corpus; `cpu_baseline`: the oracle's C++ restatement of kgram.rs's
query-filtered counting on this host, on a bounded prefix of the same workload (a tenth of the corpus and of the
queries)."""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "n-gram-hinted-lm_amd"))

HBM_PEAK_GBS = 8000.0
# the count path: the level scans, the bitmap-to-list of sparse levels, the region packing, the partition sort and the
# LDS counts; its algorithmic bytes are the build's 2 per position read + 16 per hit
PATH_KERNELS = ("scan_emit", "bits_list", "gather", "partition", "count")
TRAFFIC = ROOT / "profiles" / "scan_traffic_c3.json"  # rocprofv3 FETCH_SIZE / WRITE_SIZE of the scans, per level


def measured_traffic(k: int):
    """HBM bytes per launch of level k's scan from the committed rocprofv3 counter runs (FETCH_SIZE and WRITE_SIZE
    scaled by a plain copy's reading of them), with the commit they were taken at; None where there is none."""
    if not TRAFFIC.exists():
        return None, None
    t = json.loads(TRAFFIC.read_text())
    v = t.get("bytes_per_launch", {}).get(str(k))
    return v, t.get("commit")


def measured_fetch(k: int):
    """The scaled FETCH_SIZE of level k's scan per launch from the same counter runs (bytes read beyond L2), or None."""
    if not TRAFFIC.exists():
        return None
    return json.loads(TRAFFIC.read_text()).get("fetch_bytes_per_launch", {}).get(str(k))


def roof(nbytes: float, msec: float) -> dict:
    """Achieved GB/s of nbytes in msec milliseconds against MI355X's HBM peak."""
    gbs = nbytes / (msec / 1e3) / 1e9 if msec > 0 else 0.0
    return {"achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS}


def median_runs(fn, runs: int = 3) -> dict:
    """fn() once untimed (a warm-up: pages touched, caches filled), then `runs` timed runs: their median and range."""
    import statistics

    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return {"median_s": statistics.median(ts), "runs_s": ts}


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", default="c3", choices=("c3",), help="the headline workload")
    ap.add_argument("--train-tokens", type=int, default=0, help="override the corpus size (smaller runs)")
    ap.add_argument("--query-tokens", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-secondary", action="store_true", help="skip the other configurations' measurements")
    ap.add_argument("--only", default="", choices=("", "c1", "c2", "c4", "c5", "copy", "load"),
                    help="measure only this secondary configuration and print its JSON (for profiling); copy: three "
                         "plain 1 GiB device copies, the calibration of rocprofv3's FETCH_SIZE / WRITE_SIZE; load: "
                         "c3 from shard files (the threaded loader, and the build overlapped with the copies)")
    ap.add_argument("--cpu-tokens", type=int, default=100_000_000, help="CPU baseline and parity: corpus prefix")
    ap.add_argument("--cpu-queries", type=int, default=1_600_000, help="CPU baseline and parity: query positions")
    ap.add_argument("--parity-windows", type=int, default=400,
                    help="windows of 64 query positions compared against the oracle over the whole corpus (0: none)")
    return ap.parse_args()


def log(*a) -> None:
    print(*a, file=sys.stderr, flush=True)


def make_workload(cfg_name: str, train_tokens: int, query_tokens: int):
    """The configuration's corpus laid out in shards on the GPU and its query stream (both generated on the GPU)."""
    import numpy as np
    import torch

    from ngram_amd import data

    t0 = time.time()
    dc = data.device_corpus(cfg_name, train_tokens or None, query_tokens or None)
    torch.cuda.synchronize()
    log(f"workload on the GPU: {time.time() - t0:.1f}s")
    return dc.config, dc.flat, dc.bounds, dc.tok, dc.sizes, dc.starts, dc.query, np


def bench_c2(steps: int, warmup: int, with_cpu: bool) -> dict:
    """Configuration c2: a corpus-wide CountTable over a 100M-token corpus for n = 2..4, then the
    top-4 continuations (with counts), tot / dist / cnt of 8M query positions; one step = build + query."""
    import numpy as np
    import torch

    from ngram_amd.count_table import CountTable

    cfg, flat, bounds, tok, sizes, starts, q, _ = make_workload("c2", 0, 0)
    x, tgt = q[:-1], q[1:]
    levels = list(cfg.levels)
    ct0 = CountTable.from_device(tok, sizes, starts, levels)
    from ngram_amd.count_table import _segments_device

    avail = _segments_device(x, ct0.lib)
    times = []
    sizing = None  # the warm steps size their tables from the last build (its contexts and pairs per occurrence)
    cold_ms = None
    for step in range(warmup + steps):
        ct = CountTable.from_device(tok, sizes, starts, levels, sizing=sizing)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ct.build()
        r = ct.query_device(x, tgt, avail, topk=cfg.topk)
        torch.cuda.synchronize()
        if step == 0:
            cold_ms = (time.perf_counter() - t0) * 1e3
        if step >= warmup:
            times.append(time.perf_counter() - t0)
        sizing = ct.sizing
        sizes_out = ct.sizes()
        ev = {}
        for name, k, e0, e1 in ct.events:
            ev[name] = ev.get(name, 0.0) + e0.elapsed_time(e1)
        del ct, r
    dt = sum(times) / len(times)
    T = sum(sizes)
    res = {"value": T / dt, "unit": "corpus tokens/s", "query_positions_per_s": x.numel() / dt, "ms_per_step": dt * 1e3,
           "workload": f"c2: CountTable of {T} corpus tokens for n={levels} + top-{cfg.topk}/tot/dist/cnt queries at "
                       f"{x.numel()} positions", "kernel_ms_per_step": ev,
           "sizes": [list(v) for v in sizes_out],
           "cold": {"first_build_ms": cold_ms, "is": "the first step: sizes from the occurrences alone (nothing learned), "
                                                    "first in this process"}}
    # B_build = 2 T + 16 E with E = T x L (every corpus position is an event at every level, within shard edges)
    E = T * len(levels)
    build_bytes = 2.0 * T + 16.0 * E
    res["build_bytes"] = build_bytes
    res["roofline"] = {"bound": "hbm", "kernel": "whole step (CountTable.build + query_device)",
                       "algorithmic_bytes_per_step": build_bytes, "events_per_step": E, **roof(build_bytes, dt * 1e3),
                       "dominant_class": max(ev, key=ev.get), "dominant_ms_per_step": max(ev.values())}
    if with_cpu:
        sys.path.insert(0, str(ROOT / "oracle"))
        import oracle as O

        # the whole configuration (100M tokens x 8M queries, every level), median of three after a warm-up run
        train = flat.cpu().numpy().view(np.uint16)
        qq = q.cpu().numpy().view(np.uint16)
        xs, ts = qq[:-1], qq[1:]
        av = O.segments(xs)
        b = np.array([0, len(train)], np.int64)
        cdt = median_runs(lambda: [O.table_counts(train, b, xs, ts, av, k, ntop=4, nthreads=O.threads())
                                   for k in levels])
        res["cpu_baseline"] = {"value": T / cdt["median_s"], "unit": "corpus tokens/s", "cores": O.threads(),
                               "kind": "port", "query_positions_per_s": len(xs) / cdt["median_s"],
                               "sample": f"the whole configuration: count_table.rs restatement over {T} tokens x "
                                         f"{len(xs)} queries, levels {levels}; median of 3 after a warm-up",
                               **cdt}
    return res


def bench_c1(steps: int, warmup: int, with_cpu: bool) -> dict:
    """Configuration c1, whole: a 4M-token corpus (four shards of 2^20) and 256K query positions; per position and
    level k = 2, 3 its tot / dist / cnt and top-1 next token with its count (CountBuild), and its longest exact
    suffix match up to 32 with the next token and count there (longest_match). One step = both over the resident
    corpus. With with_cpu: the oracle on the same whole configuration (median of 3 after a warm-up), and every output
    compared with it."""
    import numpy as np
    import torch

    from ngram_amd import data
    from ngram_amd.counts import CountBuild, device_queries
    from ngram_amd.lib import Lib
    from ngram_amd.longest import _segments, longest_match

    dc = data.device_corpus("c1")
    levels = (2, 3)
    cb = CountBuild.from_device(dc.tok, dc.sizes, dc.starts, levels=levels, level_shards={}, topk=1)
    x, tgt, avail = device_queries(dc.query)
    lib = Lib()
    seg = _segments(x, lib)
    times = []
    for step in range(warmup + steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out = cb.counts(x, tgt, avail)
        length, nxt, cnt, _ = longest_match(dc.tok, x, seg, 32, elib=lib, lib=lib)
        torch.cuda.synchronize()
        if step >= warmup:
            times.append(time.perf_counter() - t0)
    dt = sorted(times)[len(times) // 2]
    T, N = sum(dc.sizes), x.numel()
    res = {"value": T / dt, "unit": "corpus tokens/s", "query_positions_per_s": N / dt, "ms_per_step": dt * 1e3,
           "workload": f"c1: counts (n={list(levels)}, top-1) and the longest suffix match (cap 32) of {N} query "
                       f"positions against {T} corpus tokens", "steps": steps, "statistic": "median step"}
    if with_cpu:
        sys.path.insert(0, str(ROOT / "oracle"))
        import oracle as O

        train = dc.flat.cpu().numpy().view(np.uint16)
        q = dc.query.cpu().numpy().view(np.uint16)
        xs, ts = q[:-1], q[1:]
        av = O.segments(xs)
        b = np.asarray(dc.bounds, np.int64)
        got = {}

        def cpu():
            for k in levels:
                got[k] = O.query_counts(train, b, xs, ts, av, k, cnt_top=1 << 30, ntop=1, nthreads=O.threads())
            got["long"] = O.longest_match(train, b, xs, av, 32, nthreads=O.threads())

        cdt = median_runs(cpu)
        res["cpu_baseline"] = {"value": T / cdt["median_s"], "unit": "corpus tokens/s",
                               "query_positions_per_s": N / cdt["median_s"], "cores": O.threads(), "kind": "port",
                               "sample": "the whole configuration (kgram.rs counts for n = 2, 3 and the longest-match "
                                         "ladder, cap 32); median of 3 after a warm-up", **cdt}
        o = out.cpu().numpy()
        bad = 0
        for li, k in enumerate(levels):
            w = got[k]
            bad += int(((o[0, li].view(np.uint32) != w["tot"]) | (o[1, li].astype(np.uint16) != w["dist"])
                        | (o[2, li].view(np.uint32) != w["cnt"])
                        | (cb.top_tok[li, :, 0].cpu().numpy().view(np.uint16) != w["top_tok"][:, 0])
                        | (cb.top_cnt[li, :, 0].cpu().numpy().view(np.uint32) != w["top_cnt"][:, 0])).sum())
        ln, nx, cn = got["long"][:3]
        bad += int(((length.cpu().numpy().view(np.uint32) != ln) | (nxt.cpu().numpy().view(np.uint16) != nx)
                    | (cnt.cpu().numpy().view(np.uint32) != cn)).sum())
        res["parity"] = {"positions": N, "mismatching_positions": bad}
    return res


def bench_c5(tok, flat, steps: int, warmup: int, with_cpu: bool) -> dict:
    """Configuration c5 over the c3 corpus already in `tok` (`flat`: its tokens without gaps): a
    held-out 64M-token stream (15% of documents with a copied span of 16-2048 corpus tokens), queried at every
    fourth position (16M positions): the longest exact suffix match (cap 64), its top next token and count."""
    import numpy as np
    import torch

    from ngram_amd import data
    from ngram_amd.lib import Lib
    from ngram_amd.longest import _segments, longest_match

    c3 = data.CONFIGS["c3"]
    zipf, tp, _ = data.make_plans(c3)
    n = 64_000_000 + 1
    qp = data.make_plan(data.stream_key("c5", "query", n), n, copy_rate=0.15, copy_len=(16, 2048), source=tp)
    lib = Lib()
    q = data.realize_gpu(qp, zipf, lib, source=flat)
    x = q[:-1]
    avail = _segments(x, lib)
    query = torch.zeros(x.numel(), dtype=torch.bool, device=x.device)
    query[3::4] = True
    nq = int(query.sum().item())
    times, timing = [], {}
    for step in range(warmup + steps):
        timing.clear()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        length, nxt, cnt, ladder = longest_match(tok, x, avail, 64, timing=timing, query=query)
        torch.cuda.synchronize()
        if step >= warmup:
            times.append(time.perf_counter() - t0)
    dt = sum(times) / len(times)
    T = int(flat.numel())
    hist = torch.bincount(length[query].long(), minlength=65).cpu().tolist()
    E = int(timing.get("events", 0))
    build_bytes = 2.0 * T + 16.0 * E
    res = {"value": T / dt, "unit": "corpus tokens/s", "query_positions_per_s": nq / dt, "ms_per_step": dt * 1e3,
           "workload": f"c5: longest exact suffix match (cap 64) + top next token and count of {nq} positions of a "
                       f"64M-token held-out stream against {T} corpus tokens", "phases_s": dict(timing),
           "levels": len(ladder), "length_histogram": hist,
           # B_build = 2 T + 16 E, E the (context, next) events the counting phase counts (the final contexts' hits)
           "roofline": {"bound": "hbm", "kernel": "whole step (existence + counting phases)",
                        "algorithmic_bytes_per_step": build_bytes, "events_per_step": E,
                        **roof(build_bytes, dt * 1e3),
                        "counting_phase": {"algorithmic_bytes": 16.0 * E,
                                           **roof(16.0 * E, 1e3 * timing.get("count", 0.0))}}}
    if with_cpu:
        sys.path.insert(0, str(ROOT / "oracle"))
        import oracle as O

        n_t, n_q = 100_000_000, 200_000
        train = flat[:n_t].cpu().numpy().view(np.uint16)
        xs = x[: 4 * n_q].cpu().numpy().view(np.uint16)
        av = O.segments(xs)
        cdt = median_runs(lambda: O.longest_match(train, np.array([0, n_t], np.int64), xs, av, 64,
                                                  nthreads=O.threads()))
        res["cpu_baseline"] = {"value": n_t / cdt["median_s"], "unit": "corpus tokens/s", "cores": O.threads(),
                               "kind": "port", **cdt,
                               "sample": f"kgram.rs-style ladder over the first {n_t} corpus tokens x {4 * n_q} "
                                         f"contiguous query positions, cap 64 (a tenth of the corpus); median of 3 "
                                         f"after a warm-up"}
    return res


def bench_c4(with_cpu: bool) -> dict:
    """Configuration c4: 92 steps of 2^19 fresh tokens (copied-span rate ramping 0 -> 20%); each step
    answers its 2^19 queries (hint rows at n = 2..6: the deepest level with a count, 8 next tokens and weights, and
    count rows tot / dist / cnt per level) from the occurrences of earlier steps, its own occurrences becoming
    available to the next step (OnlineRows.advance, the step rule). Per-step latency over all 92 steps."""
    import numpy as np
    import torch

    from ngram_amd import data
    from ngram_amd.lib import Lib
    from ngram_amd.online import OnlineRows

    zipf, plan, spans = data.c4_stream()
    tok = data.realize_gpu(plan, zipf, Lib()).cpu().numpy().view(np.uint16)
    n = len(tok)
    levels = [2, 3, 4, 5, 6]
    buckets = [2, 3, 4, 5, 6, 10, 20]
    rows = OnlineRows(tok, [0, n], spans)
    rows.prepare(levels, buckets, 8, levels)
    # one untimed pass over a copy of the state warms the allocator and the kernels
    warm = OnlineRows(tok, [0, n], spans)
    warm.prepare(levels, buckets, 8, levels)
    warm.advance_device(4)
    torch.cuda.synchronize()
    del warm
    lat = []
    for s in range(len(spans)):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        rows.advance_device(s + 1)
        torch.cuda.synchronize()
        lat.append(time.perf_counter() - t0)
    rows._check_flags(rows.state)
    lat_ms = np.array(lat) * 1e3
    step_tokens = int(spans[0, 1] - spans[0, 0])
    # per step: E = step_tokens x levels insert events (2 T + 16 E) and its queries (N (2 + 8 L) + N L 29)
    E = step_tokens * len(levels)
    step_bytes = 2.0 * step_tokens + 16.0 * E + step_tokens * (2 + 8 * len(levels)) + step_tokens * len(levels) * 29
    res = {"value": n / sum(lat), "unit": "stream tokens/s (insert + query)", "steps": len(spans),
           "roofline": {"bound": "hbm", "kernel": "whole step (insert, merge, query, hint rows)",
                        "algorithmic_bytes_per_step": step_bytes, **roof(step_bytes, float(lat_ms.mean())),
                        "note": "latency-bound: 2^19 tokens a step leave the chip mostly idle"},
           "step_tokens": step_tokens, "ms_per_step_mean": float(lat_ms.mean()),
           "ms_per_step_median": float(np.median(lat_ms)), "ms_per_step_p99": float(np.percentile(lat_ms, 99)),
           "ms_per_step_max": float(lat_ms.max()),
           "workload": f"c4: OnlineRows.advance over {len(spans)} steps x {step_tokens} tokens, hint rows (n={levels}, "
                       f"8 entries) + count rows per step"}
    if with_cpu:
        sys.path.insert(0, str(ROOT / "oracle"))
        import oracle as O

        # the whole stream, every step's rows, by the oracle's batch walk (one thread per host core)
        tau, tau_in = O.spans_tau(n, [0, n], spans)
        cores = O.threads()
        t0 = time.perf_counter()
        O.online(tok, [0, n], tau, tau_in, levels, buckets, 8, levels, 0, len(spans), nthreads=cores)
        cdt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": n / cdt, "unit": "stream tokens/s (insert + query)", "cores": cores,
                               "kind": "port", "sample": f"online.rs step-rule walk (oracle_online) over all "
                                                         f"{len(spans)} steps ({n} tokens); {cdt:.1f} s"}
    return res


def bench_load(cfg, tok, sizes, starts, q, steps: int) -> dict:
    """The host data path at c3: the shards written as shard files to tmpfs (untimed), then (1) the threaded loader
    (preadv into pinned staging buffers, per-thread copy streams) into a fresh token buffer, checked against the
    resident one; (2) CountBuild from the files (read into pinned host memory before the clock), each step
    start_load() + counts(): every shard's copy enqueued, each level's scan of a shard waiting for that shard's copy,
    against the same build over already resident tokens."""
    import shutil
    import tempfile

    import numpy as np
    import torch

    from ngram_amd import data
    from ngram_amd.counts import CountBuild, device_queries
    from ngram_amd.loader import Loader

    need = 2 * sum(sizes) * 1.2
    shm = Path("/dev/shm")
    root = shm if shm.is_dir() and shutil.disk_usage(shm).free > need else None
    d = Path(tempfile.mkdtemp(prefix="ngram_load_", dir=root))
    try:
        paths = []
        for i, (st, n) in enumerate(zip(starts, sizes)):
            p = d / f"train_{i:06d}.bin"
            data.write_shard(p, tok[st : st + n].cpu().numpy().view(np.uint16))
            paths.append(str(p))
        threads = min(16, len(os.sched_getaffinity(0)))
        res: dict = {"shards": len(paths), "bytes": 2 * sum(sizes), "threads": threads, "files": str(root or "tmp")}
        loads = []
        for _ in range(2):
            ld = Loader(paths, tok.numel(), starts, sizes, threads, chunk_tokens=8 << 20, start=False)
            ld.preallocate()
            torch.cuda.synchronize()
            ld.start()
            ld.join()
            assert torch.equal(ld.tok, tok), "the loaded buffer differs from the resident one"
            loads.append(ld.stats["seconds"])
            del ld
        res["loader_s"] = min(loads)
        res["loader_GBps"] = res["bytes"] / min(loads) / 1e9
        cb = CountBuild(paths, levels=cfg.levels, level_shards={}, topk=cfg.topk)
        x, tgt, avail = device_queries(q, cb.lib)
        cb.start_load(1)
        want = cb.counts(x, tgt, avail, stats=True).clone()  # the levels' densities, as the headline's first build
        resident, overlapped, load_ms = [], [], []
        for _ in range(steps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out = cb.counts(x, tgt, avail)
            torch.cuda.synchronize()
            resident.append(time.perf_counter() - t0)
            cb.tok.fill_(-1)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            cb.start_load(1)
            out = cb.counts(x, tgt, avail)
            torch.cuda.synchronize()
            overlapped.append(time.perf_counter() - t0)
            load_ms.append(cb.load_ms())
            assert torch.equal(out, want), "the build over loaded shards differs"
        res.update(resident_ms=1e3 * min(resident), with_load_ms=1e3 * min(overlapped),
                   copies_ms=min(load_ms), copies_GBps=res["bytes"] / (min(load_ms) / 1e3) / 1e9,
                   tokens_per_s_with_load=sum(sizes) / min(overlapped))
        return res
    finally:
        shutil.rmtree(d, ignore_errors=True)


def cpu_baseline(flat_host, bounds, q_host, levels, n_tokens: int, n_queries: int):
    """The oracle's query-filtered counting (C++ restatement of kgram.rs, one thread per core) over a bounded sample
    of the same workload: the corpus' first n_tokens tokens and the first n_queries query positions, every level,
    tot / dist / cnt + top-4 (no TOP rule, as the record). Returns (the baseline's JSON, the outputs per level)."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O

    train = flat_host[:n_tokens].numpy().view(np.uint16)
    b = [int(v) for v in bounds if v < n_tokens] + [n_tokens]
    qq = q_host[: n_queries + 1].numpy().view(np.uint16)
    x, tgt = qq[:-1], qq[1:]
    avail = O.segments(x)
    cores = O.threads()
    outs = {}

    def run():
        for k in levels:
            outs[k] = O.query_counts(train, np.array(b, np.int64), x, tgt, avail, k, cnt_top=1 << 30, ntop=4,
                                     nthreads=cores)

    cdt = median_runs(run)
    dt = cdt["median_s"]
    return {"value": n_tokens / dt, "unit": "corpus tokens/s", "query_positions_per_s": n_queries / dt,
            "cores": cores, "kind": "port", **cdt,
            "sample": f"first {n_tokens} corpus tokens x first {n_queries} query positions (a tenth of each: the "
                      f"whole 1B x 16M would take minutes of host time per run), levels {list(levels)}, tot/dist/cnt "
                      f"+ top-4; median of 3 after a warm-up", "seconds": dt}, outs


def _mismatches(gpu: dict, want, sel=None) -> int:
    """Positions where any of tot / dist / cnt / top-4 differs (sel: the positions compared)."""
    import numpy as np

    bad = np.zeros(len(want["tot"]) if sel is None else int(sel.sum()), bool)
    for name in ("tot", "dist", "cnt", "top_tok", "top_cnt"):
        w = want[name][:, :4] if name.startswith("top") else want[name]
        w = w if sel is None else w[sel]
        d = gpu[name] != w
        bad |= d if d.ndim == 1 else d.any(1)
    return int(bad.sum())


def parity_prefix(cfg, flat, q, n_tokens: int, n_queries: int, want: dict) -> dict:
    """The GPU build over the CPU baseline's sample (the first n_tokens corpus tokens, one shard, and the first
    n_queries query positions) against the oracle's outputs on it: mismatching positions per level."""
    import numpy as np
    import torch

    from ngram_amd import data
    from ngram_amd.counts import CountBuild, device_queries

    starts, length = data.pack_layout([n_tokens])
    tok = torch.full((length,), -1, dtype=torch.int16, device=flat.device)
    tok[starts[0] : starts[0] + n_tokens].copy_(flat[:n_tokens])
    cb = CountBuild.from_device(tok, [n_tokens], starts, levels=cfg.levels, level_shards={}, topk=4)
    x, tgt, avail = device_queries(q[: n_queries + 1])
    out = cb.counts(x, tgt, avail).cpu().numpy()
    tt, tc = cb.top_tok.cpu().numpy().view(np.uint16), cb.top_cnt.cpu().numpy().view(np.uint32)
    per = {}
    for li, k in enumerate(cfg.levels):
        gpu = {"tot": out[0, li].view(np.uint32), "dist": out[1, li].astype(np.uint16),
               "cnt": out[2, li].view(np.uint32), "top_tok": tt[li], "top_cnt": tc[li]}
        per[str(k)] = _mismatches(gpu, want[k])
    return {"positions": n_queries, "corpus_tokens": n_tokens, "levels": len(per),
            "mismatching_positions": sum(per.values()), "per_level": per}


def parity_windows(cfg, flat, q, out, top_tok, top_cnt, windows: int) -> dict:
    """Windows of 64 consecutive query positions (random ones, and ones at the hottest level-2 contexts), their
    outputs from the timed build compared with the oracle's over the whole corpus (each level examining only the
    corpus positions the previous level hit)."""
    import numpy as np

    from ngram_amd import data

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O

    t0 = time.perf_counter()
    qq = q.cpu().numpy().view(np.uint16)
    x, tgt = qq[:-1], qq[1:]
    av = O.segments(x)
    N = len(x)
    rng = np.random.default_rng(2026)
    hot = np.argsort(out[0, 0].view(np.uint32))[-max(1, windows // 8) :]
    starts = np.unique(np.clip(np.concatenate([rng.integers(0, N, windows), hot - 32]), 7, N - 64))
    idx = (starts[:, None] + np.arange(-7, 64)[None, :]).reshape(-1)
    cmp = np.tile(np.arange(-7, 64) >= 0, len(starts))
    s_av = np.where(cmp, av[idx], 0).astype(np.int32)
    train = flat.cpu().numpy().view(np.uint16)
    b = np.array(data.train_bounds(len(train), cfg.shard_tokens), np.int64)
    g = idx[cmp]
    per, gate = {}, None
    for li, k in enumerate(cfg.levels):
        o = O.query_counts(train, b, x[idx], tgt[idx], s_av, k, cnt_top=1 << 30, ntop=4, hits=True, gate=gate)
        gate = o["hits"]
        gpu = {"tot": out[0, li, g].view(np.uint32), "dist": out[1, li, g].astype(np.uint16),
               "cnt": out[2, li, g].view(np.uint32), "top_tok": top_tok[li, g], "top_cnt": top_cnt[li, g]}
        per[str(k)] = _mismatches(gpu, o, cmp)
    return {"positions": int(cmp.sum()), "corpus_tokens": len(train), "windows": len(starts),
            "mismatching_positions": sum(per.values()), "per_level": per,
            "oracle_seconds": time.perf_counter() - t0}


def probe_roof(k: int, probes: int, msec: float, gather: dict, profiled: bool = True) -> dict:
    """The probe roofline of level k's scan: its 128-byte line requests beyond L2 per second (the committed FETCH_SIZE
    of the launch over 128 B, for the profiled workload), else its probes per second, against `gather`'s rate."""
    fetch = measured_fetch(k) if profiled else None
    sec = msec / 1e3
    probes_s = probes / sec / 1e9 if sec > 0 else 0.0
    if fetch is None or sec <= 0:
        achieved, what = probes_s, "probes"
    else:
        achieved, what = fetch / 128 / sec / 1e9, "line requests beyond L2 (FETCH_SIZE / 128 B)"
    return {"achieved": achieved, "peak": gather["rate"], "unit": "G requests/s", "frac": achieved / gather["rate"],
            "achieved_is": what, "probes_per_launch": probes, "probes_per_s": probes_s * 1e9,
            "calibration": gather}


def gather_rate(slots: int, loads: int = 1 << 28) -> dict:
    """The rate of random 8-byte loads from a table of `slots` u64 (ng_gather_probe: the level scans' probe pattern
    alone), best of three timed launches after a warm one: the probe roofline's peak."""
    import torch

    from ngram_amd.lib import Lib, i32, u64

    lib = Lib()
    grid = torch.cuda.get_device_properties(0).multi_processor_count * 32
    table = torch.zeros(max(slots, 1), dtype=torch.int64, device="cuda")
    out = torch.empty(grid * 256, dtype=torch.int64, device="cuda")
    best = float("inf")
    for rep in range(4):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        lib("ng_gather_probe", table, u64(table.numel()), u64(loads), u64(rep + 1), i32(grid), out)
        e1.record()
        e1.synchronize()
        if rep:
            best = min(best, e0.elapsed_time(e1))
    del table, out
    return {"table_bytes": 8 * max(slots, 1), "loads": loads, "ms": best, "rate": loads / (best / 1e3) / 1e9}


def main() -> None:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs one GPU only (got --gpus {args.gpus}): this build has no multi-GPU path", file=sys.stderr)
        sys.exit(2)
    import torch

    from ngram_amd.counts import CountBuild, device_queries

    torch.cuda.set_device(0)
    if args.only == "copy":
        a = torch.ones(1 << 27, dtype=torch.int64, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"config": "copy", "bytes_read": a.numel() * 8, "bytes_written": b.numel() * 8, "copies": 3}))
        return
    if args.only in ("c1", "c2", "c4"):
        r = bench_c2(args.steps, args.warmup, not args.no_cpu) if args.only == "c2" else \
            bench_c1(args.steps, args.warmup, not args.no_cpu) if args.only == "c1" else bench_c4(not args.no_cpu)
        r.pop("sizes", None)
        print(json.dumps({"config": args.only, **r}))
        return
    cfg, flat, bounds, tok, sizes, starts, q, np = make_workload(args.config, args.train_tokens, args.query_tokens)
    if args.only == "c5":
        print(json.dumps({"config": "c5", **bench_c5(tok, flat, args.steps, args.warmup, not args.no_cpu)}))
        return
    if args.only == "load":
        del flat
        print(json.dumps({"config": "c3 load", **bench_load(cfg, tok, sizes, starts, q, args.steps)}))
        return
    T = sum(sizes)
    x, tgt, avail = device_queries(q)
    N = x.numel()
    # cold builds: the process's first (module loads and the allocator's growth included), then a fresh engine that
    # has learnt nothing (its query tables, partitions and lists sized from their own first reads)
    cold = {}
    for label in ("first_in_process_ms", "cold_ms"):
        cb = CountBuild.from_device(tok, sizes, starts, levels=cfg.levels, level_shards={}, topk=cfg.topk)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        cb.counts(x, tgt, avail)
        torch.cuda.synchronize()
        cold[label] = 1e3 * (time.perf_counter() - t0)
    cold["reruns"] = cb.engine.reruns
    log("cold:", json.dumps(cold))
    # one untimed build with hit counts: the hits E of the roofline (deterministic, the same every step)
    cb.counts(x, tgt, avail, stats=True)
    info = {k: dict(v) for k, v in cb.info.items()}
    log("levels:", json.dumps(info))
    for _ in range(max(0, args.warmup - 1)):
        cb.counts(x, tgt, avail)
    torch.cuda.synchronize()
    reruns0 = cb.engine.reruns
    torch.cuda.reset_peak_memory_stats()
    per_kernel: dict[tuple, float] = {}  # (name, level) -> ms over the timed steps
    modes: dict[int, int] = {}
    t0 = time.perf_counter()
    t_last = t0
    step_events = []  # each step's launch events, read after the clock stops
    for step in range(args.steps):
        out = cb.counts(x, tgt, avail)
        torch.cuda.synchronize()
        now = time.perf_counter()
        log(f"step {step}: {1e3 * (now - t_last):.1f} ms")
        t_last = now
        step_events.append(cb.kernel_events)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    peak_alloc, peak_reserved = torch.cuda.max_memory_allocated(), torch.cuda.max_memory_reserved()
    # query-side hits H: (position, level) pairs whose context occurred (dist > 0)
    H = int((out[1] > 0).sum().item())
    for events in step_events:
        for name, k, n, e0, e1, mode in events:
            per_kernel[(name, k)] = per_kernel.get((name, k), 0.0) + e0.elapsed_time(e1)
            if name == "scan_emit":
                modes[k] = mode
    ms = dt / args.steps * 1e3
    hits = {k: info[k]["hits"] for k in cfg.levels}
    # positions each level's scan probes (the gate's set positions: the previous level's hits, under the prefix rule
    # where it applies), and those whose tokens it reads: every position (dense) or the probed ones (listed)
    probed = {k: info[k]["probed"] for k in cfg.levels}
    read = {k: T if modes.get(k, 0) == 0 else probed[k] for k in cfg.levels}
    scan_bytes = {k: 2.0 * read[k] + 8.0 * hits[k] for k in cfg.levels}
    scan_ms = {k: per_kernel.get(("scan_emit", k), 0.0) / args.steps for k in cfg.levels}
    dom = max(cfg.levels, key=lambda k: scan_ms[k])
    top_class = max(per_kernel, key=per_kernel.get)

    # the committed counters describe the default workload (c3 at its stated size) only
    profiled = not args.train_tokens and not args.query_tokens
    traffic, traffic_commit = measured_traffic(dom) if profiled else (None, None)
    gather = gather_rate(int(info[dom]["ids"]))
    path_ms = sum(v for (name, _), v in per_kernel.items() if name in PATH_KERNELS) / args.steps
    path_bytes = sum(2.0 * read[k] + 16.0 * hits[k] for k in cfg.levels)
    E = sum(hits.values())
    build_bytes = 2.0 * T + 16.0 * E  # the count build's B_build = 2 T + 16 E
    nl = len(cfg.levels)
    q_bytes = N * (2.0 + 8.0 * nl) + H * 6.0 * cfg.topk + N * nl * 29.0
    q_ms = sum(v for (name, _), v in per_kernel.items() if name in ("qindex", "pos_gather")) / args.steps
    classes: dict[str, float] = {}
    for (name, _), v in per_kernel.items():
        classes[name] = classes.get(name, 0.0) + v / args.steps
    res = {
        "metric": "corpus tokens counted/s + hint queries/s on 1 GPU; % of HBM peak GB/s",
        "value": T * args.steps / dt,
        "unit": "corpus tokens/s",
        "query_positions_per_s": N * args.steps / dt,
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u16/u64 (integer)",
        "data": "synthetic (seeded Zipf(1.1) documents with copied spans, generated on the GPU)",
        "config": {"workload": f"{cfg.name}: count build of {T} corpus tokens ({len(sizes)} shards) for n="
                               f"{list(cfg.levels)} + top-{cfg.topk}/count/hit queries at {N} positions",
                   "corpus_tokens": T, "query_positions": N, "levels": list(cfg.levels), "topk": cfg.topk},
        "roofline": {"bound": "hbm", "kernel": f"scan_emit k={dom} (ng_scan_emit, mode {modes.get(dom, 0)})",
                     **roof(scan_bytes[dom], scan_ms[dom]), "traffic": traffic,
                     "traffic_source": None if traffic is None else f"profiles/scan_traffic_c3.json @ {traffic_commit}",
                     # the line traffic the kernel moves beyond L2 (FETCH_SIZE x 2 + WRITE_SIZE of the same launch,
                     # from the profile) over its time here: a random 8-byte probe costs a 128-byte line beyond L2.
                     # FETCH_SIZE counts every request past L2, Infinity-Cache (MALL) hits included, so this is not
                     # HBM traffic alone
                     "traffic_is": "beyond L2 (MALL hits included)",
                     "beyond_l2_GBps": None if traffic is None else traffic / (scan_ms[dom] / 1e3) / 1e9,
                     "beyond_l2_frac_of_hbm_peak": None if traffic is None else
                     traffic / (scan_ms[dom] / 1e3) / 1e9 / HBM_PEAK_GBS,
                     "algorithmic_bytes_per_launch": scan_bytes[dom], "avg_launch_ms": scan_ms[dom],
                     "positions_read": read[dom], "hits_emitted": hits[dom],
                     "bytes_per_position_read": 2, "bytes_per_hit": 8},
        # the scans' own bound: random lines from a table beyond L2, against the rate the chip sustains for random
        # 8-byte loads from a table of the dominant level's size (ng_gather_probe, measured here: one line request
        # each). achieved: the scan's line requests beyond L2 (its FETCH_SIZE from the same commit's counters, in
        # 128-byte lines) per second; a probe that hits L2 (the hot contexts of a Zipf stream) costs no request, so
        # probes per second alone can exceed the uniform-random rate
        "probe_roofline": {"bound": "random lines beyond L2", "kernel": f"scan_emit k={dom}",
                           **probe_roof(dom, probed[dom], scan_ms[dom], gather, profiled)},
        "roofline_family": {"kernels": "scan_emit, every level", **roof(sum(scan_bytes.values()),
                                                                        sum(scan_ms.values())),
                            "ms_per_step": sum(scan_ms.values())},
        "count_path_roofline": {"kernels": list(PATH_KERNELS), "algorithmic_bytes_per_step": path_bytes,
                                "ms_per_step": path_ms, **roof(path_bytes, path_ms)},
        "build_roofline": {"bytes": build_bytes, **roof(build_bytes, ms), "streaming_floor_GBps": 2.0 * T / (ms / 1e3) / 1e9},
        "slowest_launch_class": {"kernel": f"{top_class[0]} k={top_class[1]}", "ms_per_step": per_kernel[top_class] / args.steps},
        # the query side's algorithmic bytes B_query: the query indexes (2 B per position + an 8-byte key per level) and
        # the per-position outputs (H hits' top-k records read, 6 B per entry; 29 B written per position and level)
        "query_roofline": {"kernels": ["qindex", "pos_gather"], "hits": H,
                           "algorithmic_bytes_per_step": q_bytes, "ms_per_step": q_ms, **roof(q_bytes, q_ms)},
        "cold": cold,
        "peak_mem_gb": peak_alloc / 1e9, "peak_reserved_gb": peak_reserved / 1e9,
        "reruns_in_timed_steps": cb.engine.reruns - reruns0,
        "kernel_ms_per_step": classes,
        "events_per_step": E,
        "host_s_per_step": {k: v / (args.steps + args.warmup) for k, v in cb.engine.host_s.items()},
        "levels": {str(k): {**info[k], "scan_mode": modes.get(k, 0), "positions_read": read[k],
                            "scan_ms": scan_ms[k], "probes_per_s": probed[k] / max(scan_ms[k], 1e-9) * 1e3}
                   for k in cfg.levels},
        "parity": None,
        "cpu_baseline": None,
    }
    out_np = out.cpu().numpy()
    tt_np, tc_np = cb.top_tok.cpu().numpy().view(np.uint16), cb.top_cnt.cpu().numpy().view(np.uint32)
    del cb, out, x, tgt, avail
    torch.cuda.empty_cache()
    parity = {}
    if not args.no_cpu:
        nt = min(args.cpu_tokens, int(flat.numel()))
        nq = min(args.cpu_queries, N)
        cpu, want = cpu_baseline(flat[:nt].cpu(), bounds, q[: nq + 1].cpu(), cfg.levels, nt, nq)
        log(f"cpu baseline: {cpu['seconds']:.1f}s")
        res["cpu_baseline"] = cpu
        parity["prefix"] = parity_prefix(cfg, flat, q, nt, nq, want)
        del want
    if args.parity_windows:
        parity["windows"] = parity_windows(cfg, flat, q, out_np, tt_np, tc_np, args.parity_windows)
        log(f"parity windows: {parity['windows']['oracle_seconds']:.1f}s")
    if parity:
        parity["mismatching_positions"] = sum(p["mismatching_positions"] for p in parity.values())
        res["parity"] = parity
    if not args.no_secondary:
        # the same build with every shard copied from pinned host memory inside the step (PCIe included; `value`
        # above is the resident-token figure)
        log("pcie-inclusive c3")
        res["pcie_inclusive"] = bench_load(cfg, tok, sizes, starts, q, 2)
        res["pcie_inclusive"]["unit"] = "corpus tokens/s (tokens_per_s_with_load: shards copied inside the step)"
        del q
        torch.cuda.empty_cache()
        res["secondary"] = {}
        log("secondary: c1")
        res["secondary"]["c1"] = bench_c1(5, 1, not args.no_cpu)
        torch.cuda.empty_cache()
        log("secondary: c5")
        res["secondary"]["c5"] = bench_c5(tok, flat, 2, 1, not args.no_cpu)
        del flat, tok
        torch.cuda.empty_cache()
        log("secondary: c2")
        res["secondary"]["c2"] = bench_c2(2, 1, not args.no_cpu)
        torch.cuda.empty_cache()
        log("secondary: c4")
        res["secondary"]["c4"] = bench_c4(not args.no_cpu)
    print(json.dumps(res), flush=True)
    c1p = res.get("secondary", {}).get("c1", {}).get("parity")
    if c1p and c1p["mismatching_positions"]:
        log("parity: the GPU's c1 outputs differ from the oracle's")
        sys.exit(1)
    if res["parity"] and res["parity"]["mismatching_positions"]:
        log("parity: the GPU's outputs differ from the oracle's")
        sys.exit(1)


if __name__ == "__main__":
    main()
