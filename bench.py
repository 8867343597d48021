"""Benchmark: exact kNN QPS of the MI355X FlatIndex backend.

Workload (the headline): FlatIndex exact L2 over 1,000,000 x 128 fp32 SIFT-like integers
in [0, 255] (clipped exponential, mean ~20), 10,000 queries of the same distribution,
k = 10, synthetic and seeded. One step = one search_batch of the 10,000 queries with the
queries already resident in HBM and results written to HBM (px_flat_search_device).

Prints one JSON line. roofline.achieved = 2 * nq * N * D flop per scan launch divided by
the scan kernel's mean duration, timed with HIP events on the library's stream around
every timed launch. cpu_baseline times the CPU oracle (a C restatement of the reference's
per-query scan, flat.rs:106-148 with distance.rs:3-39) on a bounded query sample on the
host's cores, and the same sample checks parity of the GPU results.

  python bench.py [--steps K] [--warmup W] [--workload flat|pq|copy] [--config 1|2|3|5]
                  [--k K] [--n N] [--nq NQ] [--mask] [--cpu-seconds S] [--gpus 1]
                  [--envelope PATH]

--envelope also writes the run as a results envelope in the reference's artefact format
(schema_version 1, provenance, workload, results; crates/core/examples/gpu_knn.rs:274-333,
bench/results/gpu.json) for the flat and PQ workloads.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from proxima_amd import FlatIndex, Metric, PqIndex, _lib, datagen  # noqa: E402

FP32_MFMA_PEAK_TFLOPS = 157.3   # MI355X dense fp32 matrix peak
FP16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 matrix peak
HBM_PEAK_GBS = 8000.0           # MI355X HBM3E


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Dev:
    """Device buffers through the library's own HIP runtime (no second runtime)."""

    def __init__(self):
        self.lib = _lib.load()
        self.ptrs = []

    def put(self, arr: np.ndarray) -> ctypes.c_void_p:
        p = ctypes.c_void_p()
        rc = self.lib.px_dev_alloc(ctypes.byref(p), max(arr.nbytes, 16))
        if rc:
            raise RuntimeError(_lib.last_error())
        self.ptrs.append(p)
        if arr.nbytes and self.lib.px_dev_upload(p, arr.ctypes.data, arr.nbytes):
            raise RuntimeError(_lib.last_error())
        return p

    def empty(self, nbytes: int) -> ctypes.c_void_p:
        p = ctypes.c_void_p()
        if self.lib.px_dev_alloc(ctypes.byref(p), max(nbytes, 16)):
            raise RuntimeError(_lib.last_error())
        self.ptrs.append(p)
        return p

    def get(self, p, arr: np.ndarray) -> np.ndarray:
        if self.lib.px_dev_download(arr.ctypes.data, p, arr.nbytes):
            raise RuntimeError(_lib.last_error())
        return arr

    def free(self):
        for p in self.ptrs:
            self.lib.px_dev_free(p)
        self.ptrs = []


def host_cpu() -> dict:
    """The host the CPU baseline ran on: usable CPUs (affinity) and the CPU model."""
    model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        nproc = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        nproc = os.cpu_count() or 1
    return {"nproc": nproc, "cpu_model": model}


def cpu_baseline(data, queries, k, metric, gpu_ids, gpu_d, budget_s, mask=None, pq=None,
                 warm_mt=64, warm_st=8, single=True, max_queries=None):
    """The oracle (the reference's per-query scan restated in C, one query per OpenMP task
    as rayon's par_chunks_mut in flat.rs:173-181) timed as bench/harness.py:256-265 times
    the reference: a 64-query warmup, then the median of 7 timed batches. Done twice, on all
    the host's OpenMP threads and on one thread, each within about budget_s / 2 of CPU
    time: the batch size comes from the warmup's rate. The 7 batches of each mode are
    consecutive, distinct query chunks, and every query timed is also checked against the
    GPU's results (ids exact, distances relative). warm_mt / warm_st: the warmups (queries);
    single=False skips the one-thread mode; max_queries bounds the sample to the first
    queries of the batch (a corpus too large to stream many queries through in seconds)."""
    import oracle

    nq = len(queries) if max_queries is None else min(len(queries), max_queries)

    def run(qs, threads):
        t0 = time.perf_counter()
        if pq is None:
            r = oracle.flat_search(data, qs, k, metric, mask=mask, nthreads=threads)
        else:
            books, codes = pq
            r = oracle.pq_search(books, codes, qs, k, metric, mask=mask, nthreads=threads)
        return time.perf_counter() - t0, r

    par = {"queries_checked": 0, "id_mismatches": 0, "max_rel_dist_err": 0.0}
    seen = set()

    def check(rows, o_ids, o_d):
        g_ids, g_d = gpu_ids[rows], gpu_d[rows]
        par["queries_checked"] += len(rows)
        seen.update(int(r) for r in rows)
        par["distinct_queries"] = len(seen)
        par["id_mismatches"] += int((g_ids != o_ids).sum())
        ok = o_ids >= 0
        if ok.any():
            r = np.abs(g_d[ok] - o_d[ok]) / np.maximum(np.abs(o_d[ok]), 1e-30)
            par["max_rel_dist_err"] = max(par["max_rel_dist_err"], float(r.max()))

    nxt = 0  # next query of the batch to time (chunks wrap round a short batch)

    def chunk(size):
        nonlocal nxt
        rows = (nxt + np.arange(size)) % nq
        nxt = (nxt + size) % nq
        return rows

    def mode(threads, warm, share):
        rows = chunk(warm)
        t, _ = run(queries[rows], threads)
        per_query = t / warm
        size = int(max(8, min(nq, (budget_s * share / 7.0) / max(per_query, 1e-9))))
        times = []
        for _ in range(7):
            rows = chunk(size)
            t, (o_ids, o_d, _) = run(queries[rows], threads)
            times.append(t)
            check(rows, o_ids, o_d)
        med = float(np.median(times))
        return size / med, size, med

    threads = oracle.max_threads()
    mt_qps, mt_size, mt_med = mode(threads, min(warm_mt, nq), 0.5 if single else 1.0)
    host = host_cpu()
    out = {"value": mt_qps, "unit": "queries/s", "cores": threads, "kind": "port",
           "sample": f"median of 7 batches of {mt_size} queries ({mt_med:.2f} s each) after "
                     f"a {min(warm_mt, nq)}-query warmup, full corpus, {threads} OpenMP threads"
                     + (f", queries drawn from the first {nq} of the batch"
                        if nq < len(queries) else ""),
           "host": {**host, "omp_threads": threads}}
    if single:
        st_qps, st_size, st_med = mode(1, min(warm_st, nq), 0.5)
        out["single_thread"] = {"value": st_qps, "unit": "queries/s", "cores": 1,
                                "sample": f"median of 7 batches of {st_size} queries "
                                          f"({st_med:.2f} s each) after a "
                                          f"{min(warm_st, nq)}-query warmup"}
    return out, par


def read_traffic(name: str, default_workload: bool):
    """HBM bytes per launch (calibrated FETCH_SIZE + WRITE_SIZE) from the committed rocprofv3
    summary of this workload; None when the run is not that workload or no summary exists."""
    path = os.path.join(ROOT, "profiles", name)
    if not name or not default_workload or not os.path.isfile(path):
        return None
    with open(path) as fh:
        for line in fh:
            if line.startswith("hbm_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    return None


def read_counters(name: str, default_workload: bool):
    """The `key: value` figures (mfma_busy_frac, lds_busy_frac, shader_clock_ghz, ...) of a
    committed rocprofv3 counter summary of this workload; None when the run is not that
    workload or no summary exists."""
    path = os.path.join(ROOT, "profiles", name)
    if not name or not default_workload or not os.path.isfile(path):
        return None
    out = {}
    with open(path) as fh:
        for line in fh:
            key, sep, val = line.partition(":")
            if sep and key.replace("_", "").isalnum() and key == key.lower() and " " not in key:
                try:
                    out[key] = float(val)
                except ValueError:
                    pass
    out["source"] = f"profiles/{name}"
    return out


# rocprofv3 counter summaries (MFMA busy of the scan; LDS busy of the PQ scan), by the same
# keys as TRAFFIC_PROFILES
COUNTER_PROFILES = {
    (3, 1_000_000, 10_000, 10, "collect-bounded"):
        "flat_collect_scan_bounded_l2_1Mx128_q10k_k10_mfma_counters.md",
    (3, 1_000_000, 10_000, 100, "collect-sampled"): "flat_collect_scan_l2_1Mx128_q10k_k100.md",
    (2, 100_000, 1_000, 10, "lists"): "flat_list16q_kernel_ip_100kx384_q1k_k10_mfma_counters.md",
    (5, 10_000_000, 16_384, 100, "collect-sampled"):
        "flat_collect_scan_ip_10Mx384_q16k_k100_mask10_mfma_counters.md",
}
# the PQ scan's (traffic, counter) summaries, unfiltered and with the 50% filter
PQ_PROFILES = {
    False: ("pq_scan_kernel_l2_1Mx16_q10k_k10.md", "pq_scan_kernel_l2_1Mx16_q10k_k10_lds_counters.md"),
    True: ("pq_scan_kernel_l2_1Mx16_q10k_k10_mask50.md",
           "pq_scan_kernel_l2_1Mx16_q10k_k10_mask50_lds_counters.md"),
}


# bench/harness.py:21-23: single-query latency samples and the seed of their picks
LATENCY_SAMPLES = 10_000
LATENCY_SEED = 20240917


def single_query_latency(index, queries, k, samples, batch_ids):
    """Single-query latency as bench/harness.py:238-253 measures it: `samples` calls of
    index.search on one query each (from a numpy row: upload, search, download and the Python
    surface's checks), the queries picked at random (seeded), each call timed on its own;
    p50, p99 and mean in ms. One untimed call first (the handle's one-query workspace). Every
    call's ids are compared with the batch search's afterwards."""
    rng = np.random.default_rng(LATENCY_SEED)
    picks = rng.integers(0, len(queries), size=samples)
    times = np.empty(samples, dtype=np.float64)
    got = np.empty((samples, k), dtype=np.int64)
    index.search(queries[picks[0]], k=k)
    for i, qi in enumerate(picks):
        q = queries[qi]
        t0 = time.perf_counter()
        ids, _ = index.search(q, k=k)
        times[i] = (time.perf_counter() - t0) * 1e3
        got[i] = ids
    same = bool(np.array_equal(got, batch_ids[picks]))
    out = {"p50_ms": float(np.percentile(times, 50)), "p99_ms": float(np.percentile(times, 99)),
           "mean_ms": float(times.mean()), "samples": int(samples), "seed": LATENCY_SEED,
           "form": "index.search(query, k) from a numpy row, one call per query",
           "same_ids_as_batch_search": same}
    log(f"[bench] single-query latency over {samples} calls: p50 {out['p50_ms']:.3f} ms, "
        f"p99 {out['p99_ms']:.3f} ms, mean {out['mean_ms']:.3f} ms, same ids {same}")
    return out


def host_buffer_qps(search, nq, reps=7):
    """Median of `reps` timed calls of a search from host (numpy) arrays after one warmup:
    query upload, the device pipeline, result download and the Python surface's checks,
    as the reference's harness times search_batch (bench/harness.py:256-265)."""
    out = search()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        out = search()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {"value": nq / med, "unit": "queries/s", "ms_median": med * 1e3, "reps": reps,
            "warmup": 1}, out


# rocprofv3 summaries whose calibrated FETCH_SIZE + WRITE_SIZE give `traffic`, by
# (workload, rows, queries, k, path that ran); other runs report null
TRAFFIC_PROFILES = {
    (3, 1_000_000, 10_000, 10, "lists"): "flat_scan_kernel_l2_1Mx128_q10k_k10.md",
    (3, 1_000_000, 10_000, 10, "collect-bounded"): "flat_collect_scan_bounded_l2_1Mx128_q10k_k10.md",
    (3, 1_000_000, 10_000, 100, "collect-sampled"): "flat_collect_scan_l2_1Mx128_q10k_k100.md",
    (2, 100_000, 1_000, 10, "lists"): "flat_list16q_kernel_ip_100kx384_q1k_k10.md",
    (5, 10_000_000, 16_384, 100, "collect-sampled"):
        "flat_collect_scan_ip_10Mx384_q16k_k100_mask10.md",
}

# the same for the fp16 collect scan (rows and queries exact in fp16), by the same keys
F16_PROFILES = {
    (3, 1_000_000, 10_000, 10, "collect-bounded"): "flat_collect_scan_f16_l2_1Mx128_q10k_k10.md",
}

HEADLINE_METRIC = "exact kNN QPS (1M\u00d7128 fp32, k=10, 10k-query batch); % fp32 MFMA / HBM peak"


def bench_flat(args, dev):
    """FlatIndex search_batch on one of the flat workloads (datagen.CONFIGS 1, 2, 3, 5);
    workload 3 (1M x 128 SIFT-like integers, L2, 10k queries, k=10) is the headline."""
    c = args.config
    cfg = datagen.CONFIGS[c]
    if cfg["kind"] != "flat":
        raise SystemExit(f"workload {c} is not a FlatIndex workload")
    gt = None
    if args.sift:
        # SIFT1M from its TEXMEX files (bench/bench_sift.py:44-60): L2, recall against the
        # published ground truth
        from proxima_amd import datasets

        ds = datasets.load_sift(args.sift)
        data = np.ascontiguousarray(ds.base[: args.n] if args.n else ds.base)
        queries = np.ascontiguousarray(ds.queries[: args.nq] if args.nq else ds.queries)
        if len(data) == len(ds.base):
            gt = ds.ground_truth[: len(queries)]
        cfg = dict(cfg, dist="sift1m", metric="L2", mask=None)
        n, dim = data.shape
        nq = len(queries)
        k = args.k or 10
        l2 = True
        log(f"[bench] SIFT1M from {args.sift}: base {n} x {dim}, {nq} queries")
    else:
        n = args.n or cfg["n"]
        nq = args.nq or cfg["nq"]
        k = args.k or cfg["k"][0]
        dim = cfg["dim"]
        l2 = cfg["metric"] == "L2"
        log(f"[bench] workload {c}: generating corpus {n} x {dim} ({cfg['dist']}) and {nq} queries")
        data = datagen.corpus(c, rows=n)
        queries = datagen.queries(c, rows=nq)
    mask = datagen.config_mask(c, n) if cfg["mask"] is not None else None
    n_eff = int(mask.sum()) if mask is not None else n
    idx = FlatIndex(dim, Metric.L2 if l2 else Metric.InnerProduct)
    t0 = time.perf_counter()
    idx.add(data)
    log(f"[bench] add + upload {time.perf_counter() - t0:.2f} s")
    lib = dev.lib
    dq = dev.put(queries)
    dm = dev.put(mask.view(np.uint8)) if mask is not None else None
    di = dev.empty(nq * k * 8)
    dd = dev.empty(nq * k * 4)

    # the search and its timing read bound once: per step one library call for the search
    # and one for the HIP-event times it recorded (kernel and pipeline)
    search, search_args = lib.px_flat_search_device, (idx._h, dq, nq, k, dm, di, dd)
    ev_scan, ev_total, ev_splits, ev_blocks = (ctypes.c_float(), ctypes.c_float(),
                                               ctypes.c_int(), ctypes.c_int())
    read_timing = lib.px_flat_last_timing
    timing_args = (idx._h, ctypes.byref(ev_scan), ctypes.byref(ev_total),
                   ctypes.byref(ev_splits), ctypes.byref(ev_blocks))

    def step():
        if search(*search_args):
            raise RuntimeError(_lib.last_error())

    def timed_loop(steps, warmup, events):
        """warmup steps, then steps timed by the host clock. events: each search also records
        the library's HIP events (an opt-in diagnostic whose markers sit between its
        kernels), read after it for the kernel and pipeline times."""
        idx._timing(events)
        for _ in range(warmup):
            step()
        scan, total = [], []
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
            if events:
                read_timing(*timing_args)
                scan.append(ev_scan.value)
                total.append(ev_total.value)
        return time.perf_counter() - t0, scan, total

    # the metric is the fp32 scan's: the fp16 scan (rows and queries exact in fp16) is timed
    # after it, as its own object of the line. value and ms_per_step: the searches as a
    # caller makes them; the kernel and pipeline times: the same searches again with the HIP
    # events on (on workload 2 they add ~1% a search)
    idx._scan_f16(False)
    elapsed, _, _ = timed_loop(args.steps, args.warmup, False)
    _, scan_ms, total_ms = timed_loop(args.steps, 1, True)
    info = idx._last_timing()
    idx._timing(False)  # the host-buffer and latency measurements below without the events
    log(f"[bench] {args.steps} steps in {elapsed:.3f} s; scan {np.mean(scan_ms):.3f} ms, "
        f"pipeline {np.mean(total_ms):.3f} ms, splits {info['splits']}, blocks {info['blocks']}")
    ids = dev.get(di, np.empty((nq, k), dtype=np.int64))
    dists = dev.get(dd, np.empty((nq, k), dtype=np.float32))
    # the same batch from host arrays through the Python surface (FlatIndex.search_batch)
    if mask is not None:
        hb, (h_ids, h_d) = host_buffer_qps(lambda: idx.search_batch_filtered(queries, mask, k=k), nq)
    else:
        hb, (h_ids, h_d) = host_buffer_qps(lambda: idx.search_batch(queries, k=k), nq)
    hb["same_results_as_device_form"] = bool(np.array_equal(h_ids, ids) and
                                              np.array_equal(h_d.view(np.uint32),
                                                             dists.view(np.uint32)))
    log(f"[bench] host-buffer search_batch: {hb['ms_median']:.3f} ms median of 7, "
        f"{hb['value']:.0f} QPS")
    latency = None
    if args.latency > 0 and mask is None:
        latency = single_query_latency(idx, queries, k, args.latency, ids)

    # the same searches with the collect scan multiplying in fp16, where every value of the
    # rows and queries is exact in fp16 (the products are then exact either way)
    f16 = None
    if not args.no_f16:
        idx._scan_f16(True)
        el16, _, _ = timed_loop(args.steps, max(args.warmup, 1), False)
        _, scan16, total16 = timed_loop(args.steps, 1, True)
        info16 = idx._last_timing()
        idx._timing(False)
        if info16["scan_f16"]:
            ids16 = dev.get(di, np.empty((nq, k), dtype=np.int64))
            d16 = dev.get(dd, np.empty((nq, k), dtype=np.float32))
            fl16 = 2.0 * nq * n_eff * dim / (np.mean(scan16) * 1e-3) / 1e12
            f16 = {"value": nq * args.steps / el16, "unit": "queries/s",
                   "dtype": "f16 operands (every value exact in fp16), f32 accumulation; "
                            "f32 re-rank",
                   "ms_per_step": el16 / args.steps * 1e3,
                   "kernel_ms": float(np.mean(scan16)), "pipeline_ms": float(np.mean(total16)),
                   "achieved_tflops": fl16, "peak_tflops": FP16_MFMA_PEAK_TFLOPS,
                   "frac": fl16 / FP16_MFMA_PEAK_TFLOPS, "collect_rounds": info16["collect_rounds"],
                   "traffic": read_traffic(F16_PROFILES.get((c, n, nq, k, info16["path"]), ""),
                                           not args.sift),
                   "same_results_as_fp32_scan": bool(
                       np.array_equal(ids16, ids) and
                       np.array_equal(d16.view(np.uint32), dists.view(np.uint32)))}
            # from host arrays through the Python surface, as host_buffer above
            if mask is not None:
                hb16, (hi16, hd16) = host_buffer_qps(
                    lambda: idx.search_batch_filtered(queries, mask, k=k), nq)
            else:
                hb16, (hi16, hd16) = host_buffer_qps(lambda: idx.search_batch(queries, k=k), nq)
            hb16["same_results_as_device_form"] = bool(
                np.array_equal(hi16, ids16) and np.array_equal(hd16.view(np.uint32), d16.view(np.uint32)))
            f16["host_buffer"] = hb16
            log(f"[bench] fp16 scan: {f16['ms_per_step']:.3f} ms a batch, {f16['value']:.0f} QPS, "
                f"scan {f16['kernel_ms']:.3f} ms, same results {f16['same_results_as_fp32_scan']}; "
                f"host-buffer {hb16['ms_median']:.3f} ms")
            ctr16 = read_counters(F16_PROFILES.get((c, n, nq, k, info16["path"]), ""), not args.sift)
            if ctr16 and "mfma_busy_frac" in ctr16:
                f16["mfma_busy"] = {"frac": ctr16["mfma_busy_frac"],
                                    "lds_busy_frac": ctr16.get("lds_busy_frac"),
                                    "source": ctr16["source"]}
        idx._scan_f16(False)

    flops = 2.0 * nq * n_eff * dim
    # rows of exactly 128 padded dims take flat_collect_kernel, rows of 129-384 the collect
    # mode of flat_list16q_kernel (the threshold sample's dense scan staying on
    # flat_scan_kernel), other widths the collect mode of flat_scan_kernel
    dp_ = (dim + 7) // 8 * 8
    collect_kernel = ("flat_collect_kernel" if dp_ == 128 else
                      "flat_list16q_kernel" if 128 < dp_ <= 384 else "flat_scan_kernel")
    # lists of 32 (k + 8 <= 32) over rows of 129-384 padded dims take flat_list16q_kernel (the
    # queries resident in registers), other lists flat_scan_kernel
    list_kernel = ("flat_list16q_kernel" if k + 8 <= 32 and 128 < (dim + 7) // 8 * 8 <= 384
                   else "flat_scan_kernel")
    achieved = flops / (np.mean(scan_ms) * 1e-3) / 1e12
    headline = (c, n, nq, k) == (3, 1_000_000, 10_000, 10) and not args.sift
    desc = (f"FlatIndex exact {'L2' if l2 else 'inner product'}, corpus {n} x {dim} fp32 "
            f"{ {'gaussian': 'N(0,1)', 'unit': 'unit-normalised Gaussian', 'sift': 'SIFT-like integers in [0,255]', 'sift1m': 'SIFT1M base vectors'}[cfg['dist']] }, "
            f"{nq}-query batch, k={k}" + (f", {cfg['mask']:.0%}-density filter" if mask is not None else ""))
    result = {
        "metric": HEADLINE_METRIC if headline else f"exact kNN QPS ({desc}); % fp32 MFMA peak",
        "value": nq * args.steps / elapsed,
        "unit": "queries/s",
        "ms_per_step": elapsed / args.steps * 1e3,
        "dtype": "f32",
        "config": {"workload": desc, "n": n, "dim": dim, "nq": nq, "k": k,
                   "metric": "L2" if l2 else "IP", "mask_density": cfg["mask"],
                   "n_eff": n_eff, "queries_resident_in_hbm": True},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": FP32_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": achieved / FP32_MFMA_PEAK_TFLOPS,
                     "traffic": read_traffic(TRAFFIC_PROFILES.get((c, n, nq, k, info["path"]), ""),
                                             not args.sift),
                     "kernel": {"lists": f"{list_kernel} (per-split lists)",
                                "collect-sampled": f"{collect_kernel} (threshold-collect: sample "
                                                   "scan, ladder and collect scan)",
                                "collect-bounded": f"{collect_kernel} (threshold-collect: "
                                                   "collect scan bounded by the splits' shared "
                                                   "bound, no sample)",
                                "vector": "flat_vcollect_kernel (vector-ALU collect: sample "
                                          "and collect scans)",
                                "full-sort": "flat_exact_keys_kernel (every key) and a radix sort "
                                             "of them (k past the fused scans' limit)"}[info["path"]],
                     "collect_rounds": info["collect_rounds"],
                     "kernel_ms": float(np.mean(scan_ms)),
                     "algorithmic_flop_per_launch": flops},
        "pipeline_ms": float(np.mean(total_ms)),
        "host_buffer": hb,
    }
    if f16 is not None:
        result["f16_exact_scan"] = f16
    if latency is not None:
        result["latency_single_query"] = latency
    ctr = read_counters(COUNTER_PROFILES.get((c, n, nq, k, info["path"]), ""), not args.sift)
    if ctr and "mfma_busy_frac" in ctr:
        result["roofline"]["mfma_busy"] = {
            "frac": ctr["mfma_busy_frac"],
            "counter": "SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x 1024 SIMDs)",
            "mfma_flop_per_launch": ctr.get("mfma_flop_per_launch"),
            "shader_clock_ghz": ctr.get("shader_clock_ghz"),
            "source": ctr["source"]}
    if args.sift:
        from proxima_amd import datasets

        result["data"] = f"SIFT1M TEXMEX files ({args.sift})"
        if gt is not None:
            kk = min(k, gt.shape[1])
            result["recall_at_k"] = datasets.recall_at_k(ids, gt, kk)
            log(f"[bench] recall@{kk} against the published ground truth: "
                f"{result['recall_at_k']:.4f}")
    if args.cpu_seconds > 0:
        log("[bench] CPU oracle baseline + parity sample")
        import oracle

        cb, par = cpu_baseline(data, queries, k, oracle.L2 if l2 else oracle.IP, ids, dists,
                               args.cpu_seconds, mask=mask, **getattr(args, "cpu_opts", {}))
        result["cpu_baseline"] = cb
        result["parity_sample"] = par
    return result


def bench_pq(args, dev, variants=None):
    """PqIndex ADC scan (workload 4): 1M x 128 N(0,1) rows encoded as m = 16 x 8-bit codes
    (codebooks from the reference's k-means, 25 iterations on a 50,000-row sample, seed
    24301), 10,000 queries, k = 10. variants: mask settings to measure on the one trained
    index (False: unfiltered, True: the 50%-density filter); default: --mask's. Returns the
    result of the first variant, or the list of them when variants is given."""
    n, dim, m = args.n or 1_000_000, 128, 16
    nq, k = args.nq or 10_000, args.k or 10
    log(f"[bench] generating PQ corpus {n} x {dim} N(0,1), training m={m}")
    data = datagen.gaussian(n, dim, 4001)
    queries = datagen.gaussian(nq, dim, 4002)
    pq = PqIndex(dim, Metric.L2, m=m, nbits=8, train_iters=25, train_sample=50_000)
    t0 = time.perf_counter()
    pq.train(data)
    train_s = time.perf_counter() - t0
    log(f"[bench] train {train_s:.2f} s")
    t0 = time.perf_counter()
    pq.add(data)
    add_s = time.perf_counter() - t0
    log(f"[bench] encode + upload {add_s:.2f} s")
    del data
    out = []
    for masked in (variants if variants is not None else (args.mask,)):
        mask = datagen.mask(n, 0.5, 4003) if masked else None
        res = pq_measure(args, dev, pq, queries, mask, n, m, nq, k)
        res["build_seconds"] = {"train": train_s, "encode_and_upload": add_s}
        out.append(res)
        dev.free()
    if variants is None:
        return out[0]
    return out


def pq_measure(args, dev, pq, queries, mask, n, m, nq, k):
    lib = dev.lib
    dq = dev.put(queries)
    dm = dev.put(mask.view(np.uint8)) if mask is not None else None
    di = dev.empty(nq * k * 8)
    dd = dev.empty(nq * k * 4)

    # as the flat loop: the search and its timing read bound once
    search, search_args = lib.px_pq_search_device, (pq._h, dq, nq, k, dm, di, dd)
    ev_scan, ev_total, ev_splits, ev_blocks = (ctypes.c_float(), ctypes.c_float(),
                                               ctypes.c_int(), ctypes.c_int())
    read_timing = lib.px_pq_last_timing
    timing_args = (pq._h, ctypes.byref(ev_scan), ctypes.byref(ev_total),
                   ctypes.byref(ev_splits), ctypes.byref(ev_blocks))

    def step():
        if search(*search_args):
            raise RuntimeError(_lib.last_error())

    # value and ms_per_step from searches as a caller makes them, then the same searches with
    # the library's HIP events on for the kernel and pipeline times
    pq._timing(False)
    for _ in range(args.warmup):
        step()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    elapsed = time.perf_counter() - t0
    pq._timing(True)
    step()
    scan_ms, total_ms = [], []
    for _ in range(args.steps):
        step()
        read_timing(*timing_args)
        scan_ms.append(ev_scan.value)
        total_ms.append(ev_total.value)
    pq._timing(False)
    ids = dev.get(di, np.empty((nq, k), dtype=np.int64))
    dists = dev.get(dd, np.empty((nq, k), dtype=np.float32))
    if mask is not None:
        hb, (h_ids, h_d) = host_buffer_qps(lambda: pq.search_batch_filtered(queries, mask, k=k), nq)
    else:
        hb, (h_ids, h_d) = host_buffer_qps(lambda: pq.search_batch(queries, k=k), nq)
    hb["same_results_as_device_form"] = bool(np.array_equal(h_ids, ids) and
                                              np.array_equal(h_d.view(np.uint32),
                                                             dists.view(np.uint32)))
    n_eff = int(mask.sum()) if mask is not None else n
    algo_bytes = nq * (n_eff * m + ((n + 7) // 8 if mask is not None else 0)) + nq * m * 256 * 4
    achieved = algo_bytes / (np.mean(scan_ms) * 1e-3) / 1e9
    headline_shape = (n, nq, k) == (1_000_000, 10_000, 10)
    log(f"[bench] PQ scan{' (50% mask)' if mask is not None else ''}: "
        f"{elapsed / args.steps * 1e3:.3f} ms a batch, scan {np.mean(scan_ms):.3f} ms, "
        f"{achieved:.0f} GB/s algorithmic")
    result = {
        "metric": "PqIndex ADC scan QPS (1M x m=16 x 8-bit codes, k=10, 10k-query batch"
                  + (", 50%-density filter" if mask is not None else "") + "); % HBM peak",
        "value": nq * args.steps / elapsed,
        "unit": "queries/s",
        "ms_per_step": elapsed / args.steps * 1e3,
        "dtype": "f32",
        "config": {"workload": f"PqIndex ADC L2, {n} codes x m={m} x 8 bit, {nq}-query batch, "
                               f"k={k}, mask={'50%' if mask is not None else 'none'}",
                   "n": n, "m": m, "nq": nq, "k": k, "n_eff": n_eff,
                   "queries_resident_in_hbm": True},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": read_traffic(PQ_PROFILES[mask is not None][0], headline_shape),
                     "kernel": "pq_scan_kernel", "kernel_ms": float(np.mean(scan_ms)),
                     "algorithmic_bytes_per_launch": algo_bytes},
        "pipeline_ms": float(np.mean(total_ms)),
        "host_buffer": hb,
    }
    # the scan's real limit: its LUT gathers, one 16-byte LDS read per (row, 4 queries,
    # subspace), against the measured LDS read rates (profiles/lds_gather_rate.md)
    qpb = 4
    gather_bytes = ((nq + qpb - 1) // qpb) * n_eff * m * 16
    g_ach = gather_bytes / (np.mean(scan_ms) * 1e-3) / 1e9
    lds = read_counters(LDS_PROFILE, True) or {}
    result["lds_roofline"] = {
        "bound": "lds", "achieved": g_ach, "unit": "GB/s",
        "gather_bytes_per_launch": gather_bytes,
        "peak": lds.get("lds_conflict_free_gbs"),
        "frac": g_ach / lds["lds_conflict_free_gbs"] if lds.get("lds_conflict_free_gbs") else None,
        "random_gather_ceiling": lds.get("lds_random_gather_gbs"),
        "frac_of_random_gather_ceiling": (g_ach / lds["lds_random_gather_gbs"]
                                          if lds.get("lds_random_gather_gbs") else None),
        "source": lds.get("source")}
    ctr = read_counters(PQ_PROFILES[mask is not None][1], headline_shape)
    if ctr:
        result["lds_roofline"]["counters"] = {
            "lds_busy_frac": ctr.get("lds_busy_frac"),
            "bank_conflict_cycles_per_lds_cycle": ctr.get("lds_bank_conflict_per_cycle"),
            "valu_busy_frac": ctr.get("valu_busy_frac"), "source": ctr["source"]}
    if args.latency > 0 and mask is None:
        result["latency_single_query"] = single_query_latency(pq, queries, k, args.latency,
                                                              ids)
    if args.cpu_seconds > 0:
        import oracle

        cb, par = cpu_baseline(None, queries, k, oracle.L2, ids, dists, args.cpu_seconds,
                               mask=mask, pq=(pq.codebooks(), pq.codes()))
        result["cpu_baseline"] = cb
        result["parity_sample"] = par
    return result


def bench_copy(args, dev):
    """Plain streaming copy of a known byte count: the HBM reference for traffic counters
    (FETCH_SIZE / WRITE_SIZE of this kernel divided by its known bytes gives the scale)."""
    nbytes = args.copy_mib << 20
    src = dev.empty(nbytes)
    dst = dev.empty(nbytes)
    ms = ctypes.c_float()
    times = []
    for i in range(args.warmup + args.steps):
        if dev.lib.px_dev_copy_kernel(dst, src, nbytes, ctypes.byref(ms)):
            raise RuntimeError(_lib.last_error())
        if i >= args.warmup:
            times.append(ms.value)
    gbs = 2 * nbytes / (np.mean(times) * 1e-3) / 1e9
    return {"metric": "streaming copy bandwidth (read + write)", "value": gbs, "unit": "GB/s",
            "ms_per_step": float(np.mean(times)), "dtype": "f32",
            "config": {"workload": f"copy kernel, {args.copy_mib} MiB read + {args.copy_mib} MiB "
                                   "written per launch", "bytes_read": nbytes,
                       "bytes_written": nbytes},
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "traffic": 2 * nbytes,
                         "kernel": "copy_kernel", "kernel_ms": float(np.mean(times))}}


LDS_PROFILE = "lds_gather_rate.md"


def bench_lds(args, dev):
    """LDS read-rate calibration, the PQ scan's roofline: 1,024 workgroups of 512 threads read
    16-byte slots of a 64 KB LDS table, 16 reads a loop iteration as the ADC scan issues its
    gathers, with no bank conflict and at uniform random slots (the scan's pattern on uniform
    codes). value = the conflict-free rate; random_gather = the other."""
    lib = dev.lib
    blocks, iters = 1024, 2048
    rates = {}
    for random in (0, 1):
        ms, nbytes = ctypes.c_float(), ctypes.c_double()
        times = []
        for i in range(args.warmup + args.steps):
            if lib.px_dev_lds_gather(random, blocks, iters, ctypes.byref(ms), ctypes.byref(nbytes)):
                raise RuntimeError(_lib.last_error())
            if i >= args.warmup:
                times.append(ms.value)
        rates[random] = (nbytes.value / (np.mean(times) * 1e-3) / 1e9, float(np.mean(times)),
                         nbytes.value)
    info = _lib.device_info(0)
    clk = info.get("clock_khz", 0) * 1e3
    cus = info.get("cus", 0)

    def per_clk(gbs):
        return gbs * 1e9 / (clk * cus) if clk and cus else None

    log(f"[bench] LDS 16-byte reads: {rates[0][0]:.0f} GB/s conflict-free, "
        f"{rates[1][0]:.0f} GB/s at random slots")
    return {"metric": "LDS read rate, 16-byte reads from a 64 KB table, no bank conflicts",
            "value": rates[0][0], "unit": "GB/s", "ms_per_step": rates[0][1], "dtype": "f32",
            "config": {"workload": f"lds_gather_kernel, {blocks} workgroups x 512 threads x "
                                   f"{iters} x 16 reads of 16 bytes", "bytes": rates[0][2]},
            "bytes_per_clk_per_cu": per_clk(rates[0][0]),
            "random_gather": {"value": rates[1][0], "unit": "GB/s", "ms": rates[1][1],
                              "bytes_per_clk_per_cu": per_clk(rates[1][0])}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", choices=["flat", "pq", "copy", "lds"], default="flat")
    ap.add_argument("--config", type=int, default=3, choices=[1, 2, 3, 5],
                    help="flat: which FlatIndex workload (3, the headline, by default)")
    ap.add_argument("--k", type=int, default=None, help="override the workload's k")
    ap.add_argument("--no-f16", action="store_true",
                    help="flat: skip the timing of the fp16 collect scan (rows and queries "
                         "exact in fp16)")
    ap.add_argument("--n", type=int, default=None, help="override the corpus rows")
    ap.add_argument("--nq", type=int, default=None, help="override the query count")
    ap.add_argument("--copy-mib", type=int, default=1024, help="copy: MiB per launch")
    ap.add_argument("--mask", action="store_true", help="pq: 50%% filter bitmask")
    ap.add_argument("--sift", default=None,
                    help="flat: SIFT1M TEXMEX directory (sift_base.fvecs, sift_query.fvecs, "
                         "sift_groundtruth.ivecs) instead of synthetic data")
    ap.add_argument("--envelope", default=None,
                    help="also write a schema_version 1 results envelope to this path")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="CPU oracle budget for the baseline (0 disables)")
    ap.add_argument("--latency", type=int, default=None,
                    help="single-query latency samples (bench/harness.py:238-253); default "
                         f"{LATENCY_SAMPLES} on the default run's flat and PQ workloads, else 0")
    ap.add_argument("--no-extras", action="store_true",
                    help="default run: skip the other workloads measured after the headline")
    args = ap.parse_args()
    # the default invocation (the headline workload, no overrides) also measures the other
    # workloads of the scope: the PQ ADC scan with and without its filter, the 100k x 384
    # and 10M x 384 FlatIndex workloads, and single-query latency
    default_run = (args.workload == "flat" and args.config == 3 and args.k is None and
                   args.n is None and args.nq is None and args.sift is None)
    if args.latency is None:
        args.latency = LATENCY_SAMPLES if default_run and not args.no_extras else 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this backend runs the whole search on a "
              "single MI355X and has no multi-GPU path (a sharded search would split the "
              "corpus rows across GPUs and merge each shard's k best)",
              file=sys.stderr)
        sys.exit(2)
    if _lib.device_count() < 1:
        print("bench.py needs a gfx950 GPU (none visible)", file=sys.stderr)
        sys.exit(1)
    dev = Dev()
    extras = {}
    try:
        run = {"flat": bench_flat, "pq": bench_pq, "copy": bench_copy,
               "lds": bench_lds}[args.workload]
        res = run(args, dev)
        dev.free()
        if default_run and not args.no_extras:
            extras = bench_extras(args, dev)
    finally:
        dev.free()
    out = {"metric": res.pop("metric"), "value": res.pop("value"), "unit": res.pop("unit"),
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": res.pop("ms_per_step"), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": res.pop("dtype"),
           "data": res.pop("data", "synthetic (seeded SplitMix64)"),
           "config": res.pop("config")}
    out.update(res)
    out.update(extras)
    out["device"] = _lib.device_info(0)
    if args.envelope and args.workload in ("flat", "pq"):
        write_bench_envelope(args.envelope, out)
    print(json.dumps(out), flush=True)


def bench_extras(args, dev) -> dict:
    """The other workloads of the scope, each as its own object of the default run's line
    (its own QPS, kernel time and roofline fraction, CPU baseline and parity sample):
    the PQ ADC scan (workload 4) unfiltered and with its 50% filter, the headline workload at
    k = 100 (the threshold-collect path: sample scan, ladder, collect scan), FlatIndex inner
    product on 100k x 384 (workload 2: the reference's own `make bench` shape) and on
    10M x 384 with a 10% filter, k = 100 (workload 5; the CPU oracle times a sample of its
    first 128 queries, each of which streams the ~1M kept rows)."""
    import argparse

    def sub(**kw):
        a = argparse.Namespace(**vars(args))
        a.sift = a.envelope = None
        a.n = a.nq = a.k = None
        a.no_f16 = True
        for key, v in kw.items():
            setattr(a, key, v)
        return a

    extras = {}
    t0 = time.perf_counter()
    pq_u, pq_m = bench_pq(sub(workload="pq", cpu_seconds=min(args.cpu_seconds, 6.0)), dev,
                          variants=(False, True))
    extras["pq_adc_scan"] = pq_u
    extras["pq_adc_scan_mask50"] = pq_m
    log(f"[bench] PQ workloads in {time.perf_counter() - t0:.1f} s")
    t0 = time.perf_counter()
    extras["flat_l2_1Mx128_k100"] = bench_flat(
        sub(config=3, k=100, latency=0, cpu_seconds=min(args.cpu_seconds, 6.0)), dev)
    dev.free()
    log(f"[bench] workload 3 at k = 100 in {time.perf_counter() - t0:.1f} s")
    t0 = time.perf_counter()
    extras["flat_ip_100kx384"] = bench_flat(
        sub(config=2, steps=max(args.steps, 300), warmup=max(args.warmup, 30), latency=0,
            cpu_seconds=min(args.cpu_seconds, 6.0)), dev)
    dev.free()
    log(f"[bench] workload 2 in {time.perf_counter() - t0:.1f} s")
    t0 = time.perf_counter()
    extras["flat_ip_10Mx384_mask10_k100"] = bench_flat(
        sub(config=5, latency=0, cpu_seconds=min(args.cpu_seconds, 8.0),
            cpu_opts={"warm_mt": 16, "single": False, "max_queries": 128}), dev)
    dev.free()
    log(f"[bench] workload 5 in {time.perf_counter() - t0:.1f} s")
    return extras


def write_bench_envelope(path: str, out: dict) -> None:
    """The run as a gpu_knn-style envelope: per-search seconds for the whole batch, the CPU
    oracle's rate extrapolated to the batch, agreement = share of equal ids on its sample."""
    from proxima_amd import envelope

    cfg = out["config"]
    nq, k = cfg["nq"], cfg["k"]
    cb = out.get("cpu_baseline")
    par = out.get("parity_sample")
    agree = None
    if par and par["queries_checked"]:
        agree = 1.0 - par["id_mismatches"] / (par["queries_checked"] * k)
    env = envelope.gpu_envelope(
        n_base=cfg["n"], dim=cfg.get("dim", 128), n_queries=nq, k=k,
        metric=cfg.get("metric", "L2"), gpu_seconds=out["ms_per_step"] / 1e3,
        reps=out["steps"], cpu_mt_seconds=(nq / cb["value"]) if cb else None,
        topk_agreement=agree)
    env["results"]["bench_line"] = {key: out[key] for key in ("metric", "value", "unit")}
    envelope.write_envelope(path, env)
    log(f"[bench] envelope written to {path}")


if __name__ == "__main__":
    main()
