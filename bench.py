"""Benchmark of the MaxSim hot path on one MI355X.

One step = one pass of the hot path over one batch, device-resident and
enqueued on one stream (msim_int4_topk_int8q_async): int8 quantisation of the
fp32 query [4, 32, 128] (quantize_query_int8_kernel), then the int4 x int8 MFMA
MaxSim scan over the whole per-token int4 corpus (4,096 docs, 64-192 tokens
each, dim 128), whose last workgroup selects the top-10 of each batch row
(int8q_scan_kernel<8, true, true>).
Inputs are resident in HBM before timing starts; outputs stay on the device.

Prints ONE JSON line:
  value = docs scored per second = batch * num_docs / step time.
Extra fields: p50/p95 step latency from HIP events, the roofline of the scan
kernel (timed alone with HIP events on the launch stream), the MALL-cold
variant (rotating over corpus copies whose total exceeds the 256 MB Infinity
Cache), the synchronous host-API latency (numpy in / numpy out, as the
reference times) and the CPU baseline (the C oracle, one thread, bounded
sample).

`--pmc-calibrate` appends plain device copies of known size, so that a
`rocprofv3 --pmc FETCH_SIZE` (or WRITE_SIZE) run of this script carries its
own calibration; `--summarize-pmc FETCH_CSV WRITE_CSV` turns two such runs into
HBM bytes per scan launch.
"""
from __future__ import annotations

import argparse
import ctypes
import csv
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
SCAN_KERNEL = "int8q_scan_kernel<8, 1, true, false>"  # the scan (one-fma epilogue, int4 documents) with its fused top-k tail
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "int8q_scan_config2_traffic.md")
CALIBRATION_BYTES = 256 << 20  # one plain copy: reads and writes this many bytes
SCAN_BLOCK = 10  # scan launches between two events
KERNEL_STATS = os.path.join(ROOT, "profiles", "int8q_scan_config2_kernel_stats.md")
MFMA_INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
MFMA_FP4_PEAK_TOPS = 10100.0  # MI355X dense fp4 MFMA
# The achievable bound of the fused scan under its present design, from
# measured constants: a tile's 16 MFMAs at the rate of an MFMA followed by
# three VALU instructions with two waves per SIMD (bench.py --rates,
# mfma_fma3: 11.43 ns per MFMA), plus the time until a wave's first tile
# lands (median wave, per-wave s_memrealtime stamps of a timing copy of the
# kernel: 2.1 us) and the tail from the last wave's loop end to the end of
# the selection (the same stamps: 4.8 us).
MIX_NS_PER_MFMA = 11.43
RAMP_US = 2.1
TAIL_US = 4.8
# Config 3's MaxSim score launch, the same way: its loop issues 24 MFMAs per
# 16-token tile and pass (three limbs, four row blocks) with about five other
# VALU instructions each (profiles/score_kernel_config3_sq_counters.md: 4.95),
# a mix the rate tests put between mfma_fma4 (12.79 ns per MFMA) and
# mfma_fma6 (15.61 ns): 14.2 ns.  The first tile lands at 2.0 us (median
# wave, per-wave stamps) and the last wave ends its loop about 1 us before
# the launch ends.
MIX3_NS_PER_MFMA = 14.2
RAMP3_US = 2.0
TAIL3_US = 1.0


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--k", type=int, default=10)
    ap.add_argument("--cold-copies", type=int, default=10,
                    help="corpus copies rotated for the MALL-cold measurement (0 = skip)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--docs-per-wave", type=int, default=0)
    ap.add_argument("--pmc-calibrate", action="store_true",
                    help="append plain device copies of known size (PMC calibration)")
    ap.add_argument("--pack", action="store_true",
                    help="measure the device int4 packer (index build) instead of a search config")
    ap.add_argument("--rates", action="store_true",
                    help="run the instruction-rate tests (maxsim_amd/microbench/rates.hip) instead of a search config")
    ap.add_argument("--config", type=int, default=2, choices=(2, 3, 4, 5),
                    help="BASELINE configuration to measure (2 = the headline metric)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print HBM traffic per scan launch from two rocprofv3 --pmc runs and exit")
    return ap.parse_args()


def algorithmic_bytes(num_tokens: int, num_docs: int, batch: int, query_tokens: int, k: int,
                      num_blocks: int = 512) -> dict:
    """Bytes the scan kernel (with its fused top-k) must move per launch over a
    per-token int4 corpus: 64 B of int4 codes + 4 B token scale per token, 8 B
    per document offset, the quantised query (128 B codes + 4 B scale per
    query row, read once per workgroup from L2 but counted once), the 8-byte
    selection key of every (batch row, document) written once, each
    workgroup's 24-byte record per batch row written once and read once by the
    selecting workgroup, and the top-k (4 B score + 8 B id each).  The
    selection also reads back the keys of a few workgroups (those holding a
    key at or above its threshold); they are not counted."""
    corpus = 68 * num_tokens + 8 * (num_docs + 1)
    query = batch * query_tokens * (128 + 4)
    out = 8 * batch * num_docs + 2 * 24 * batch * num_blocks + 12 * batch * k
    return {"corpus": corpus, "query": query, "out": out, "total": corpus + query + out}


def _pmc_values(path: str) -> dict:
    """Counter values (KiB per dispatch) by (kernel name, counter) of one rocprofv3 counter CSV."""
    values: dict = {}
    with open(path, newline="") as fh:
        for row in csv.DictReader(fh):
            values.setdefault((row["Kernel_Name"], row["Counter_Name"]), []).append(float(row["Counter_Value"]))
    return values


def summarize_pmc(fetch_csv: str, write_csv: str) -> dict:
    """HBM bytes per scan launch: FETCH_SIZE and WRITE_SIZE (KiB per dispatch)
    of the scan kernel, each divided by what the same counter reads per byte
    for the plain device copy of CALIBRATION_BYTES in the same run (the
    largest copy dispatches; smaller copies are the run's host transfers)."""
    out = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        values = _pmc_values(path)
        scan = [v for (name, ctr), v in values.items() if SCAN_KERNEL in name and ctr == counter]
        copy = [v for (name, ctr), v in values.items() if ctr == counter and "copybuffer" in name.lower()]
        if not scan or not copy:
            raise SystemExit(f"{path}: no {SCAN_KERNEL} or copy dispatches with {counter}")
        copies = [x for v in copy for x in v]
        top = max(copies)
        calib = [x for x in copies if x >= 0.5 * top]
        copy_kib = float(np.median(calib))
        factor = copy_kib * 1024.0 / CALIBRATION_BYTES
        scan_kib = float(np.mean(scan[0]))
        out[counter] = {"scan_kib_per_dispatch": scan_kib, "scan_dispatches": len(scan[0]),
                        "copy_kib_per_dispatch": copy_kib, "copy_dispatches": len(calib),
                        "factor": factor, "bytes_per_launch": scan_kib * 1024.0 / factor}
    out["traffic_bytes_per_launch"] = out["FETCH_SIZE"]["bytes_per_launch"] + out["WRITE_SIZE"]["bytes_per_launch"]
    return out


def read_traffic() -> float | None:
    """The committed traffic figure (line 'traffic_bytes_per_launch: N'), if any."""
    try:
        with open(TRAFFIC_SUMMARY) as fh:
            for line in fh:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        return None
    return None


def read_kernel_stats_us(kernel: str) -> float | None:
    """The committed rocprofv3 average duration (us) of `kernel`, from the
    table of the config-2 kernel-stats summary, if any."""
    try:
        with open(KERNEL_STATS) as fh:
            for line in fh:
                cells = [c.strip().strip("`") for c in line.split("|")]
                if len(cells) > 3 and cells[1] == kernel:
                    return float(cells[3])
    except (OSError, ValueError):
        return None
    return None


def scan_tiles(offsets: np.ndarray) -> int:
    """16-token tiles of the scan: ceil(len / 16) per non-empty document."""
    lens = np.diff(offsets)
    return int(((lens + 15) // 16).sum())


def lscpu_fields() -> dict:
    """The host CPU as `lscpu` names it (model name, BIOS model name, family,
    model, stepping, sockets), or the /proc/cpuinfo model name without lscpu."""
    import subprocess

    keys = ("Vendor ID", "Model name", "BIOS Model name", "CPU family", "Model", "Stepping",
            "Socket(s)", "Core(s) per socket", "Thread(s) per core")
    out = {}
    try:
        text = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10,
                              env=dict(os.environ, LC_ALL="C")).stdout
        for line in text.splitlines():
            name, _, value = line.partition(":")
            if name.strip() in keys and name.strip() not in out:
                out[name.strip()] = value.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    if "Model name" not in out:
        try:
            with open("/proc/cpuinfo") as fh:
                for line in fh:
                    if line.startswith("model name"):
                        out["Model name"] = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
    return out


def host_metadata() -> dict:
    """What the run was: command, host CPU (lscpu) and core counts, GPU, ROCm."""
    cpu = lscpu_fields()
    meta = {"benchmark_command": " ".join([os.path.basename(sys.executable)] + sys.argv),
            "cpu_model": cpu.get("Model name"), "lscpu": cpu, "nproc": os.cpu_count(),
            "cpus_allowed": len(os.sched_getaffinity(0))}
    try:
        import torch

        meta.update(gpu=torch.cuda.get_device_name(0), hip=torch.version.hip, torch=torch.__version__)
    except Exception:  # noqa: BLE001 - metadata only
        pass
    return meta


def cpu_baseline(packed, query, seconds: float):
    """The C oracle (one thread) on a bounded sample of the same workload: whole
    config-2 calls (quantise + scan of every document + top-10), repeated until
    about `seconds` have passed.  The thread is pinned to one core for the
    measurement (the reference's `taskset -c 0` protocol) and unpinned after."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc

    orc.build()
    allowed = sorted(os.sched_getaffinity(0))
    core = allowed[0]
    os.sched_setaffinity(0, {core})
    try:
        docs = 0
        start = time.perf_counter()
        reps = 0
        while True:
            scores = orc.int4_int8q_scores(query, packed.values, packed.doc_offsets, token_scale=packed.token_scale)
            orc.topk(scores, 10)
            reps += 1
            docs += query.shape[0] * (packed.doc_offsets.shape[0] - 1)
            elapsed = time.perf_counter() - start
            if elapsed >= seconds:
                break
    finally:
        os.sched_setaffinity(0, set(allowed))
    return {
        "value": docs / elapsed,
        "unit": "docs scored/s",
        "cores": 1,
        "kind": "port",
        "pinned_core": core,
        "sample": f"{reps} full config-2 call(s): [{query.shape[0]},{query.shape[1]},128] query x "
                  f"{packed.doc_offsets.shape[0] - 1} docs + top-10, C oracle (oracle/maxsim_oracle.c), "
                  f"1 thread pinned to core {core}, {elapsed:.1f} s",
        "ms_per_call": 1e3 * elapsed / reps,
    }


def cpu_baseline_threads(packed, query, seconds: float):
    """The same C oracle on every host core this process may use: documents
    split into one contiguous range per thread (ctypes releases the GIL)."""
    from concurrent.futures import ThreadPoolExecutor

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc

    threads = max(1, min(len(os.sched_getaffinity(0)), 64))
    off = packed.doc_offsets
    n = off.shape[0] - 1
    bounds = np.linspace(0, n, threads + 1).astype(np.int64)

    def part(t):
        d0, d1 = int(bounds[t]), int(bounds[t + 1])
        return orc.int4_int8q_scores(query, packed.values[off[d0]:off[d1]], off[d0:d1 + 1] - off[d0],
                                     token_scale=packed.token_scale[off[d0]:off[d1]])

    reps = 0
    start = time.perf_counter()
    with ThreadPoolExecutor(threads) as pool:
        while True:
            scores = np.concatenate(list(pool.map(part, range(threads))), axis=1)
            orc.topk(scores, 10)
            reps += 1
            elapsed = time.perf_counter() - start
            if elapsed >= seconds:
                break
    return {"value": reps * query.shape[0] * n / elapsed, "unit": "docs scored/s", "cores": threads, "kind": "port",
            "sample": f"{reps} full config-2 call(s) split over {threads} threads, C oracle, {elapsed:.1f} s"}


def bench_config2(args):
    import torch

    from maxsim_amd import _maxsim_hip, synthetic
    from maxsim_amd._native import check, ptr
    from maxsim_amd.experimental import int4_to_device, pack_int4_symmetric

    if args.docs_per_wave:
        _maxsim_hip.set_docs_per_wave(args.docs_per_wave)
    cfg = synthetic.CONFIGS[2]
    corpus = synthetic.make_corpus(cfg["num_docs"], cfg["lo"], cfg["hi"])
    query_np = synthetic.make_queries(corpus, cfg["batch"])
    packed = pack_int4_symmetric(corpus.embeddings, corpus.offsets, scale_granularity="token")
    batch, qtok = query_np.shape[:2]
    num_docs, num_tokens = packed.num_docs, int(packed.doc_offsets[-1])
    k = args.k

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    resident = int4_to_device(packed)
    handle = resident.data
    query = torch.from_numpy(query_np).to(dev)
    scores = torch.empty((batch, num_docs), dtype=torch.float32, device=dev)
    top_s = torch.empty((batch, k), dtype=torch.float32, device=dev)
    top_i = torch.empty((batch, k), dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream()
    lib = handle._lib
    sptr = _maxsim_hip._stream_ptr(stream)

    def step(h):
        # quantize_query_int8_kernel -> int8q_scan_kernel (top-k in its last workgroup)
        check(lib.msim_int4_topk_int8q_async(h._h, ptr(query), batch, qtok, k, ptr(top_s), ptr(top_i), sptr))

    # Correctness gate before timing: the device top-10 equals the stable
    # order of the device scores of the separate synchronous API.
    ref_scores = handle.maxsim_batch_int8q(query_np)
    step(handle)
    torch.cuda.synchronize()
    ref_ids = np.stack([np.lexsort((np.arange(num_docs), -row))[:k] for row in ref_scores])
    assert np.array_equal(top_i.cpu().numpy(), ref_ids), "device top-k disagrees with device scores"

    # ---- timed region: K steps back to back, bracketed by synchronize.
    for _ in range(args.warmup):
        step(handle)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(handle)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = 1e3 * wall / args.steps

    # ---- per-step latency: HIP events on the launch stream around every step.
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(args.steps)]
    for i in range(args.steps):
        ev[i][0].record(stream)
        step(handle)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    step_ms = np.array([e[0].elapsed_time(e[1]) for e in ev])

    # ---- the step's scan kernel alone (with its fused top-k): quantise once
    # outside the events, then blocks of SCAN_BLOCK back-to-back launches
    # between two events on the launch stream (consecutive launches on one
    # stream start as the previous one ends, so a block's time over
    # SCAN_BLOCK is the kernel's duration).  The scoring-only launch (no
    # selection tail) is timed the same way for reference.
    check(lib.msim_int4_quantize_int8q_async(handle._h, ptr(query), batch, qtok, sptr))
    blocks = max(1, args.steps // SCAN_BLOCK)

    def block_times(launch):
        sev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(blocks)]
        for i in range(blocks):
            sev[i][0].record(stream)
            for _ in range(SCAN_BLOCK):
                launch()
            sev[i][1].record(stream)
        torch.cuda.synchronize()
        return np.array([e[0].elapsed_time(e[1]) for e in sev]) / SCAN_BLOCK

    top_i.zero_()
    scan_ms = block_times(lambda: check(lib.msim_int4_topk_quantized_async(
        handle._h, batch, qtok, k, ptr(top_s), ptr(top_i), sptr)))
    assert np.array_equal(top_i.cpu().numpy(), ref_ids), "fused scan top-k differs"
    score_ms = block_times(lambda: check(lib.msim_int4_score_int8q_async(
        handle._h, batch, qtok, ptr(scores), sptr)))
    assert np.array_equal(scores.cpu().numpy(), ref_scores), "scan scores differ between entry points"

    # The dispatch floor: a one-workgroup kernel (torch's fill of one
    # element) launched back to back on the same stream, timed the same way.
    one = torch.empty(1, dtype=torch.float32, device=dev)
    floor_ms = block_times(lambda: one.fill_(0.0))

    # the scan's workgroups: eight waves per CU (four per workgroup), at most one wave per document
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    nbytes = algorithmic_bytes(num_tokens, num_docs, batch, qtok, k, -(-min(cus * 8, num_docs) // 4))
    scan_avg_s = float(scan_ms.mean()) * 1e-3
    achieved = nbytes["total"] / scan_avg_s / 1e9
    # MFMA work of the scan: 2 * rows * tokens * 128 int8 operations.
    mfma_ops = 2.0 * batch * qtok * num_tokens * 128
    # The achievable bound: the tiles of one SIMD (two scanning waves; the
    # first workgroup's waves scan nothing) at the mix rate, plus ramp and tail.
    waves = 4 * (-(-min(cus * 8, num_docs) // 4))
    tiles_per_simd = 2.0 * scan_tiles(packed.doc_offsets) / max(1, waves - 4)
    bound_us = RAMP_US + tiles_per_simd * 16 * MIX_NS_PER_MFMA * 1e-3 + TAIL_US
    rocprof_us = read_kernel_stats_us(SCAN_KERNEL)


    # ---- MALL-cold: rotate over corpus copies whose total exceeds the 256 MB cache.
    cold = None
    cold_scan_ms = None
    if args.cold_copies > 0:
        copies = [handle] + [int4_to_device(packed).data for _ in range(args.cold_copies - 1)]
        for c in copies:
            step(c)
        torch.cuda.synchronize()
        # the scan kernel alone, each launch on the next copy (its query quantised beforehand)
        for c in copies:
            check(lib.msim_int4_quantize_int8q_async(c._h, ptr(query), batch, qtok, sptr))
        rot = [0]

        def cold_launch():
            c = copies[rot[0] % len(copies)]
            rot[0] += 1
            check(lib.msim_int4_topk_quantized_async(c._h, batch, qtok, k, ptr(top_s), ptr(top_i), sptr))

        cold_scan_ms = block_times(cold_launch)
        cev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(args.steps)]
        t1 = time.perf_counter()
        for i in range(args.steps):
            cev[i][0].record(stream)
            step(copies[i % len(copies)])
            cev[i][1].record(stream)
        torch.cuda.synchronize()
        cold_wall = time.perf_counter() - t1
        cold_step = np.array([e[0].elapsed_time(e[1]) for e in cev])
        cold = {
            "copies": len(copies),
            "resident_MB_total": round(len(copies) * nbytes["corpus"] / 1e6, 1),
            "ms_per_step": 1e3 * cold_wall / args.steps,
            "docs_per_s": batch * num_docs / cold_wall * args.steps,
            "step_ms_p50": float(np.percentile(cold_step, 50)),
        }
        del copies

    if args.pmc_calibrate:
        src = torch.empty(CALIBRATION_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # ---- synchronous host API (numpy in, numpy out) and the end-to-end
    # Reranker.search, the reference's protocol (run_cuda_step1.py:690-736):
    # 3 runs x 20 calls after 5 warm-ups, p50 / p95.
    def host_timed(call):
        for _ in range(5):
            call()
        out = []
        for _ in range(3 * 20):
            a = time.perf_counter()
            call()
            out.append(1e3 * (time.perf_counter() - a))
        return np.array(out)

    api = host_timed(lambda: handle.topk_batch_int8q(query_np, k))
    import maxsim_amd

    ids = [f"doc{i}" for i in range(num_docs)]
    index = maxsim_amd.Index.from_embeddings(ids, corpus.embeddings, corpus.offsets, mode="int4_per_token")
    reranker = maxsim_amd.Reranker(index, device="cuda", int4_query="int8")
    res = reranker.search(query_np, k=k)
    assert [[r.doc_id for r in row] for row in res] == [[ids[i] for i in row] for row in ref_ids], \
        "Reranker.search differs from the device top-k"
    search = host_timed(lambda: reranker.search(query_np, k=k))

    cpu = None if args.no_cpu_baseline else cpu_baseline(packed, query_np, args.cpu_seconds)
    cpu_all = None if args.no_cpu_baseline else cpu_baseline_threads(packed, query_np, args.cpu_seconds / 3)
    traffic = read_traffic()

    result = {
        "metric": "docs scored/sec + p50 ms per [4,32,128] query, int4 int8q full scan (1 GPU)",
        "value": batch * num_docs / (ms_per_step * 1e-3),
        "unit": "docs scored/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "p50_ms": float(np.percentile(step_ms, 50)),
        "p95_ms": float(np.percentile(step_ms, 95)),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded normalised-Gaussian corpus, maxsim_amd/synthetic.py)",
        "config": {
            "workload": "BASELINE config 2: per-token int4 corpus, 4096 docs x U{64..192} tokens, dim 128; "
                        "query [4,32,128] quantised to int8 per token; full-corpus MaxSim + top-10",
            "num_docs": num_docs,
            "num_tokens": num_tokens,
            "batch": batch,
            "query_tokens": qtok,
            "k": k,
            "step": "quantize_query_int8_kernel + int8q_scan_kernel (top-10 selected by its last "
                    "workgroup) on one stream, device-resident (msim_int4_topk_int8q_async)",
        },
        "roofline": {
            "kernel": SCAN_KERNEL,
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "algorithmic_bytes_per_launch": nbytes["total"],
            "kernel_ms_avg": float(scan_ms.mean()),
            "kernel_ms_p50": float(np.percentile(scan_ms, 50)),
            "scoring_only_ms_avg": float(score_ms.mean()),
            "scoring_only_frac": (nbytes["total"] - 4 * batch * num_docs - 12 * batch * k)
                                 / (float(score_ms.mean()) * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "dispatch_floor_ms": float(np.median(floor_ms)),
            "mfma_frac": mfma_ops / scan_avg_s / 1e12 / MFMA_INT8_PEAK_TOPS,
            "mfma_ops_per_launch": mfma_ops,
            "rocprof_kernel_us": rocprof_us,
            "rocprof_frac": None if rocprof_us is None else nbytes["total"] / (rocprof_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "rocprof_source": "profiles/int8q_scan_config2_kernel_stats.md (rocprofv3 --kernel-trace --stats of "
                              "this script, average duration of %s; committed, not measured in this run)" % SCAN_KERNEL,
            "achievable_bound": {
                "kernel_us": bound_us,
                "frac": nbytes["total"] / (bound_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
                "tiles_per_simd": tiles_per_simd,
                "basis": "ramp %.1f us + tiles per SIMD x 16 MFMAs x %.1f ns (an MFMA and three VALU instructions, "
                         "two waves per SIMD, rate test) + tail %.1f us (last loop end to selection end); "
                         "ramp and tail from per-wave s_memrealtime stamps" % (RAMP_US, MIX_NS_PER_MFMA, TAIL_US),
            },
            "cold_kernel_ms_avg": None if cold_scan_ms is None else float(cold_scan_ms.mean()),
            "cold_frac": None if cold_scan_ms is None
                         else nbytes["total"] / (float(cold_scan_ms.mean()) * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "traffic_source": "profiles/int8q_scan_config2_traffic.md (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE "
                              "runs of this script, calibrated by a plain copy)",
            "note": "frac, mfma_frac: scan launches (with the fused top-10) back to back between HIP events on "
                    "the launch stream, averaged over blocks of %d (so each includes the launch-to-launch gap); the "
                    "35.7 MB corpus stays in the 256 MB MALL between launches (cold_*: each launch on the "
                    "next of %d corpus copies, %.0f MB in all)" % (SCAN_BLOCK, max(1, args.cold_copies),
                                                                  max(1, args.cold_copies) * nbytes["corpus"] / 1e6),
        },
        "mall_cold": cold,
        "api_sync_ms": {"p50": float(np.percentile(api, 50)), "p95": float(np.percentile(api, 95))},
        "reranker_search_ms": {"p50": float(np.percentile(search, 50)), "p95": float(np.percentile(search, 95)),
                               "calls": int(search.shape[0]),
                               "route": "maxsim_amd.Reranker(index, device='cuda', int4_query='int8').search("
                                        "query [4,32,128] numpy, k=10): H2D query, quantise + fused scan, D2H, "
                                        "SearchResult lists"},
        "cpu_baseline": cpu,
        "cpu_baseline_all_cores": cpu_all,
        "metadata": host_metadata(),
    }
    print(json.dumps(result), flush=True)

# ---------------------------------------------------------------- configs 3-5
# Secondary measurements (the driver's line is config 2).  Each returns the
# same JSON fields, with `config.workload` naming the configuration.

FP32_PEAK_TFLOPS = 157.3


def _timed(step, steps, warmup, stream):
    """Wall ms per step over `steps` back-to-back steps, and per-step event ms."""
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    wall = 1e3 * (time.perf_counter() - t0) / steps
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record(stream)
        step()
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    return wall, np.array([a.elapsed_time(b) for a, b in ev])


def _result(metric, value, unit, args, ms, p50, p95, dtype, workload, extra):
    out = {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": ms, "p50_ms": p50, "p95_ms": p95, "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": dtype,
           "data": "synthetic (seeded normalised-Gaussian corpus, maxsim_amd/synthetic.py)",
           "config": {"workload": workload}}
    out.update(extra)
    return out


def bench_config3(args):
    """fp32 query [4,32,128] x per-token int4 corpus (config-2 corpus), every
    reducer in turn; one step = full scan + device top-10 for one reducer."""
    import torch

    from maxsim_amd import _maxsim_hip, synthetic
    from maxsim_amd._native import check, ptr
    from maxsim_amd.experimental import int4_to_device, pack_int4_symmetric

    cfg = synthetic.CONFIGS[3]
    corpus = synthetic.make_corpus(cfg["num_docs"], cfg["lo"], cfg["hi"])
    query_np = synthetic.make_queries(corpus, cfg["batch"])
    weights = np.random.default_rng(synthetic.SEED + 3).uniform(0.5, 1.5, size=query_np.shape[:2]).astype(np.float32)
    packed = pack_int4_symmetric(corpus.embeddings, corpus.offsets, scale_granularity="token")
    b, q = query_np.shape[:2]
    n, t = packed.num_docs, int(packed.doc_offsets[-1])
    torch.cuda.set_device(0)
    h = int4_to_device(packed).data
    lib = h._lib
    stream = torch.cuda.current_stream()
    sptr = _maxsim_hip._stream_ptr(stream)
    dq = torch.from_numpy(query_np).cuda()
    scores = torch.empty((b, n), dtype=torch.float32, device="cuda")
    ts = torch.empty((b, args.k), dtype=torch.float32, device="cuda")
    ti = torch.empty((b, args.k), dtype=torch.int64, device="cuda")
    per = {}
    for red in ("maxsim", "weighted_maxsim", "topk2", "topk4", "smoothsim"):
        w = weights if red == "weighted_maxsim" else None
        tau = 0.7 if red == "smoothsim" else 1.0

        def step():
            check(lib.msim_int4_score_async(h._h, ptr(dq), b, q, red.encode(), ptr(w), 0 if w is None else 2,
                                            0 if w is None else b, 0 if w is None else q, tau, 0, ptr(scores), sptr))
            check(lib.msim_topk_async(ptr(scores), b, n, n, args.k, ptr(ts), ptr(ti), sptr))

        step()
        torch.cuda.synchronize()
        ref = h.score_batch(query_np, red, w, tau)
        assert np.array_equal(scores.cpu().numpy(), ref), f"{red}: device-resident scores differ from the host API"
        wall, ev = _timed(step, args.steps, args.warmup, stream)

        def score_only():
            check(lib.msim_int4_score_async(h._h, ptr(dq), b, q, red.encode(), ptr(w), 0 if w is None else 2,
                                            0 if w is None else b, 0 if w is None else q, tau, 0, ptr(scores), sptr))

        # The scoring launch alone: back-to-back launches between two events
        # on the stream (each includes the launch-to-launch gap).
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(SCAN_BLOCK * 4):
            score_only()
        e1.record(stream)
        torch.cuda.synchronize()
        kernel_ms = e0.elapsed_time(e1) / (SCAN_BLOCK * 4)
        int8_ops = 3 * 2.0 * b * q * t * 128
        per[red] = {"ms_per_step": wall, "p50_ms": float(np.percentile(ev, 50)), "docs_per_s": b * n / (wall * 1e-3),
                    "score_kernel_ms": kernel_ms,
                    "mfma_frac": int8_ops / (kernel_ms * 1e-3) / 1e12 / MFMA_INT8_PEAK_TOPS}
    # weighted MaxSim with new weights every step (two arrays alternating, so
    # the handle's unchanged-weights check never skips the upload)
    other = np.ascontiguousarray(weights[::-1])
    flip = [0]

    def fresh_step():
        w = weights if flip[0] % 2 == 0 else other
        flip[0] += 1
        check(lib.msim_int4_score_async(h._h, ptr(dq), b, q, b"weighted_maxsim", ptr(w), 2, b, q, 1.0, 0,
                                        ptr(scores), sptr))
        check(lib.msim_topk_async(ptr(scores), b, n, n, args.k, ptr(ts), ptr(ti), sptr))

    wall, ev = _timed(fresh_step, args.steps, args.warmup, stream)
    fresh = {"ms_per_step": wall, "p50_ms": float(np.percentile(ev, 50)), "docs_per_s": b * n / (wall * 1e-3),
             "note": "weighted_maxsim with different weights every step (a host-to-device copy of the weights "
                     "on the stream each step)"}
    ms = float(np.mean([v["ms_per_step"] for v in per.values()]))
    ops = 2.0 * b * q * t * 128  # multiply-adds x 2 of the fp32 contraction
    roof = {"kernel": "score_kernel (3 int8 limbs)", "bound": "mfma", "unit": "TOP/s",
            "achieved": 3 * ops / (ms * 1e-3) / 1e12, "peak": MFMA_INT8_PEAK_TOPS,
            "fp32_equivalent_TFLOPs": ops / (ms * 1e-3) / 1e12, "fp32_vector_peak_TFLOPs": FP32_PEAK_TFLOPS,
            "note": "step time (scan + top-10); int8 ops = 3 limbs x 2 B Q T 128"}
    roof["frac"] = roof["achieved"] / roof["peak"]
    # The MaxSim launch's issue bound (see MIX3_NS_PER_MFMA): two 64-row passes
    # over every tile, spread over the chip's SIMDs.
    simds = torch.cuda.get_device_properties(0).multi_processor_count * 4
    passes = (b * q + 63) // 64
    tiles_per_simd = passes * scan_tiles(packed.doc_offsets) / simds
    bound_us = RAMP3_US + tiles_per_simd * 24 * MIX3_NS_PER_MFMA * 1e-3 + TAIL3_US
    roof["maxsim_achievable_bound"] = {
        "kernel_us": bound_us, "frac": 3 * ops / (bound_us * 1e-6) / 1e12 / MFMA_INT8_PEAK_TOPS,
        "tiles_per_simd": tiles_per_simd,
        "basis": "ramp %.1f us + tiles per SIMD x 24 MFMAs x %.1f ns (an MFMA and about five VALU instructions, "
                 "two waves per SIMD, rate tests) + tail %.1f us; against the MaxSim launch's measured "
                 "score_kernel_ms" % (RAMP3_US, MIX3_NS_PER_MFMA, TAIL3_US)}
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as orc

        orc.build()
        sub = 512
        start = time.perf_counter()
        orc.int4_fp32_scores(query_np, packed.values, packed.doc_offsets[:sub + 1], token_scale=packed.token_scale)
        el = time.perf_counter() - start
        cpu = {"value": b * sub / el, "unit": "docs scored/s", "cores": 1, "kind": "port",
               "sample": f"maxsim reducer, first {sub} docs x [4,32,128] fp32 query, C oracle, 1 thread, {el:.1f} s"}
    return _result("docs scored/sec per reducer, int4 x fp32 query full scan + top-10 (1 GPU)", b * n / (ms * 1e-3),
                   "docs scored/s", args, ms, float(np.mean([v["p50_ms"] for v in per.values()])), None, "f32",
                   "BASELINE config 3: config-2 corpus, fp32 query [4,32,128], reducers maxsim / weighted (U[0.5,1.5]) "
                   "/ topk2 / topk4 / smoothsim (tau 0.7), top-10",
                   {"per_reducer": per, "weighted_maxsim_fresh_weights": fresh, "roofline": roof, "cpu_baseline": cpu})


def bench_config4(args):
    """256 sign-binarised queries x 32 tokens over 10,240 binary documents of
    256-1024 tokens; one step = all 256 queries + device top-10."""
    import torch

    from maxsim_amd import _maxsim_hip, synthetic
    from maxsim_amd._api import pack_query_signs

    cfg = synthetic.CONFIGS[4]
    lengths = synthetic.doc_lengths(cfg["num_docs"], cfg["lo"], cfg["hi"])
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    codes = np.empty((int(offsets[-1]), 16), np.uint8)
    first_tokens = []
    for first, lens, emb in synthetic.iter_blocks(cfg["num_docs"], cfg["lo"], cfg["hi"]):
        s0 = int(offsets[first])
        bits = (emb >= 0).reshape(emb.shape[0], 16, 8).astype(np.uint8)
        codes[s0:s0 + emb.shape[0]] = (bits << np.arange(8, dtype=np.uint8)).sum(axis=2, dtype=np.uint8)
        if len(first_tokens) < cfg["batch"]:
            first_tokens.append((first, lens, emb))
    rng = np.random.default_rng(synthetic.SEED + 4)
    # Queries: 32 noisy tokens of a document of the first block (the generator's recipe).
    f, lens, emb = first_tokens[0]
    loc = np.concatenate([[0], np.cumsum(lens)])
    query = np.empty((cfg["batch"], 32, 128), np.float32)
    for i in range(cfg["batch"]):
        d = int(rng.integers(0, len(lens)))
        tok = emb[loc[d]:loc[d + 1]][rng.choice(int(lens[d]), 32, replace=lens[d] < 32)]
        query[i] = tok + rng.standard_normal(tok.shape).astype(np.float32) * np.float32(0.1)
    qbits = pack_query_signs(query)
    b, q, n, t = cfg["batch"], 32, cfg["num_docs"], int(offsets[-1])
    torch.cuda.set_device(0)
    h = _maxsim_hip.CudaPackedDocs(codes, offsets, 128)
    stream = torch.cuda.current_stream()
    dq = torch.from_numpy(qbits).cuda()
    ts = torch.empty((b, args.k), dtype=torch.float32, device="cuda")
    ti = torch.empty((b, args.k), dtype=torch.int64, device="cuda")

    def step():
        h.topk_hamming_async(dq, args.k, ts, ti, stream)

    step()
    torch.cuda.synchronize()
    ref = h.hamming_batch(qbits[:8])
    # The fp4 kernel against the int8 MFMA scorer on the same rows: equal.
    _maxsim_hip.set_hamming_fp4(0)
    try:
        ref_int8 = h.hamming_batch(qbits[:8])
    finally:
        _maxsim_hip.set_hamming_fp4(1)
    assert np.array_equal(ref, ref_int8), "fp4 and int8 Hamming scores differ"
    ref_ids = np.stack([np.lexsort((np.arange(n), -row))[:args.k] for row in ref])
    assert np.array_equal(ti.cpu().numpy()[:8], ref_ids), "device top-k disagrees with device scores"
    wall, ev = _timed(step, max(3, args.steps // 20), max(1, args.warmup // 10), stream)
    ops = 2.0 * b * q * t * 128
    roof = {"kernel": "hamming_kernel (sign docs, +-1 query as fp4 on v_mfma_scale_f32_16x16x128_f8f6f4)",
            "bound": "mfma", "unit": "TOP/s", "achieved": ops / (wall * 1e-3) / 1e12, "peak": MFMA_FP4_PEAK_TOPS,
            "int8_peak_frac": ops / (wall * 1e-3) / 1e12 / MFMA_INT8_PEAK_TOPS,
            "note": "step time (scan of 8,192 query rows + top-10); ops = 2 B Q T 128 (+-1 products) against "
                    "the dense fp4 MFMA peak of the instruction used"}
    roof["frac"] = roof["achieved"] / roof["peak"]
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as orc

        ref_ext = orc.reference_cpu_extension()
        qs = np.where(query[0] >= 0, 1.0, -1.0).astype(np.float32)
        start = time.perf_counter()
        if ref_ext is not None:
            ref_ext.maxsim_lut(qs, codes, offsets, 128, 1.0)
            kind, src = "reference", "the reference's cpu_extension.cpp maxsim_lut (oracle/_ref)"
        else:
            orc.binary_lut_maxsim(qs, codes, offsets, 128)
            kind, src = "port", "C oracle binary LUT"
        el = time.perf_counter() - start
        cpu = {"value": n / el, "unit": "docs scored/s", "cores": 1, "kind": kind,
               "sample": f"1 of the 256 queries (32 tokens) x all {n} docs, {src}, 1 thread, {el:.1f} s"}
    return _result("docs scored/sec, binary sign-query XOR/popcount-equivalent full scan + top-10 (1 GPU)",
                   b * n / (wall * 1e-3), "docs scored/s", args, wall, float(np.percentile(ev, 50)),
                   float(np.percentile(ev, 95)), "fp4 (+-1)",
                   f"BASELINE config 4: {n} binary docs x U{{256..1024}} tokens ({t} tokens), 256 x 32 sign queries, "
                   "top-10",
                   {"roofline": roof, "cpu_baseline": cpu})


def bench_config5(args):
    """Binary prefix + int4 residual corpus (config-2 documents), query
    [4,32,128]: coarse scan -> top-512 -> fused rescoring -> top-10."""
    import torch

    from maxsim_amd import synthetic
    from maxsim_amd.binres import binres_to_device, pack_binary_residual

    cfg = synthetic.CONFIGS[5]
    corpus = synthetic.make_corpus(cfg["num_docs"], cfg["lo"], cfg["hi"])
    query_np = synthetic.make_queries(corpus, cfg["batch"])
    host_packed = pack_binary_residual(corpus.embeddings, corpus.offsets)
    packed = binres_to_device(host_packed)
    h = packed.sign_data
    b, q, n, t = cfg["batch"], 32, cfg["num_docs"], int(corpus.offsets[-1])
    stream = torch.cuda.current_stream()
    dq = torch.from_numpy(query_np).cuda()
    ts = torch.empty((b, args.k), dtype=torch.float32, device="cuda")
    ti = torch.empty((b, args.k), dtype=torch.int64, device="cuda")
    fs = torch.empty((b, args.k), dtype=torch.float32, device="cuda")
    fi = torch.empty((b, args.k), dtype=torch.int64, device="cuda")

    def step():
        h.cascade_topk_async(dq, args.k, 512, ts, ti, stream)

    def full():
        h.cascade_topk_async(dq, args.k, n, fs, fi, stream)

    def recall(a, e):
        return float(np.mean([len(set(a[i]) & set(e[i])) / args.k for i in range(b)]))

    wall, ev = _timed(step, args.steps, args.warmup, stream)
    full_wall, _ = _timed(full, args.steps, args.warmup, stream)
    got, exp = ti.cpu().numpy(), fi.cpu().numpy()
    overlap = recall(got, exp)
    # The same cascade with the rescoring pass on the fp32 query (three int8
    # limbs), against the fused scan of every document on the fp32 query.
    h.set_rescore_limbs(3)
    fp32_wall, _ = _timed(step, args.steps, args.warmup, stream)
    fp32_full_wall, _ = _timed(full, args.steps, args.warmup, stream)
    h.set_rescore_limbs(1)
    got32, exp32 = ti.cpu().numpy(), fi.cpu().numpy()
    cpu = None
    if not args.no_cpu_baseline:
        # The same cascade on the C oracle over the first `sub` documents,
        # with the candidate budget scaled alike (512 of 4096 -> 128 of 1024).
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as orc

        orc.build()
        sub, m_sub = 1024, 128
        off = host_packed.doc_offsets[:sub + 1]
        hp = host_packed
        start = time.perf_counter()
        coarse = orc.binres_prefix_scores(query_np, hp.sign_data, hp.prefix_scale, off)
        _, cand = orc.topk(coarse, m_sub)
        cand = np.sort(cand, axis=1)
        fine = orc.binres_fused_scores(query_np, hp.sign_data, hp.prefix_scale, hp.residual_values,
                                       hp.residual_token_scale, off, candidates=cand)
        orc.topk(fine, args.k, tie_ids=cand)
        el = time.perf_counter() - start
        cpu = {"value": b * sub / el, "unit": "docs scored/s", "cores": 1, "kind": "port",
               "sample": f"cascade over the first {sub} docs (top-{m_sub} candidates, top-{args.k}) x [4,32,128] "
                         f"query, C oracle, 1 thread, {el:.2f} s"}
    return _result("docs scored/sec, binary-prefix top-512 -> fused int4-residual rescoring -> top-10 (1 GPU)",
                   b * n / (wall * 1e-3), "docs scored/s", args, wall, float(np.percentile(ev, 50)),
                   float(np.percentile(ev, 95)), "int8",
                   f"BASELINE config 5: {n} docs ({t} tokens) as 16 B signs + 4 B prefix scale + 64 B int4 residual + "
                   "4 B residual scale per token, query [4,32,128] int8, 512 candidates, top-10",
                   {"full_fused_scan_ms_per_step": full_wall, "top10_overlap_vs_full_fused_scan": overlap,
                    "fp32_rescoring": {"ms_per_step": fp32_wall, "full_fused_scan_ms_per_step": fp32_full_wall,
                                       "top10_recall_vs_fp32_full_fused_scan": recall(got32, exp32),
                                       "int8_cascade_top10_recall_vs_fp32_full_fused_scan": recall(got, exp32)},
                    "bytes_per_token": 88, "cpu_baseline": cpu})


def bench_pack(args):
    """Index build: the config-2 corpus (fp32 [T,128], 268 MB) packed to
    per-token int4 on the device (msim_pack_int4_async, values array off).
    One step = one pack of the whole corpus, device-resident; HBM roofline
    from 512 B read + 64 B codes + 4 B scale written per token.  The host
    packer (NumPy, the reference's pack_int4_symmetric) is timed beside it."""
    import torch

    from maxsim_amd import _native, synthetic
    from maxsim_amd.experimental import pack_int4_symmetric, pack_int4_symmetric_device

    cfg = synthetic.CONFIGS[2]
    corpus = synthetic.make_corpus(cfg["num_docs"], cfg["lo"], cfg["hi"])
    x_np = np.ascontiguousarray(corpus.embeddings, np.float32)
    t, d = x_np.shape
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    x = torch.from_numpy(x_np).to(dev)
    codes = torch.empty((t, d // 2), dtype=torch.uint8, device=dev)
    tscale = torch.empty((t,), dtype=torch.float32, device=dev)
    work = torch.zeros(2, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream()
    sptr = ctypes.c_void_p(stream.cuda_stream)
    lib = _native.load()

    def step():
        _native.check(lib.msim_pack_int4_async(_native.ptr(x), t, d, 1, 0.0, _native.ptr(codes), _native.ptr(tscale),
                                               None, _native.ptr(work), sptr))

    host = pack_int4_symmetric(x_np, corpus.offsets, scale_granularity="token")
    step()
    torch.cuda.synchronize()
    assert np.array_equal(codes.cpu().numpy(), host.data), "device pack differs from the host packer"
    assert np.array_equal(tscale.cpu().numpy().view(np.uint32), host.token_scale.view(np.uint32))
    ms, ev = _timed(step, args.steps, args.warmup, stream)
    nbytes = t * (4 * d + d // 2 + 4)
    achieved = nbytes / (float(np.mean(ev)) * 1e-3) / 1e9
    h0 = time.perf_counter()
    pack_int4_symmetric(x_np, corpus.offsets, scale_granularity="token")
    host_s = time.perf_counter() - h0
    api0 = time.perf_counter()
    pack_int4_symmetric_device(x_np, corpus.offsets, scale_granularity="token")
    api_s = time.perf_counter() - api0
    tensor0 = time.perf_counter()
    tensor = pack_int4_symmetric_device(x, corpus.offsets, scale_granularity="tensor", values=False)
    tensor_s = time.perf_counter() - tensor0
    assert np.array_equal(tensor.data, pack_int4_symmetric(x_np, scale_granularity="tensor").data)
    return _result("tokens packed/sec, per-token int4 index build on the device (1 GPU)", t / (ms * 1e-3),
                   "tokens/s", args, ms, float(np.percentile(ev, 50)), float(np.percentile(ev, 95)), "f32->int4",
                   f"config-2 corpus: {t} tokens x {d} fp32 -> int4 codes + token scales",
                   {"roofline": {"kernel": "pack_int4_dim128_kernel<true>", "bound": "hbm", "achieved": achieved,
                                 "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                                 "traffic": None, "algorithmic_bytes_per_launch": nbytes},
                    "host_numpy_pack_s": host_s,
                    "api_sync_pack_s_including_transfers": api_s,
                    "tensor_scale_device_pack_s": tensor_s,
                    "cpu_baseline": {"value": t / host_s, "unit": "tokens/s", "cores": 1, "kind": "port",
                                     "sample": "one NumPy pack_int4_symmetric of the whole corpus"}})


OTHER_CONFIGS = {3: bench_config3, 4: bench_config4, 5: bench_config5}

RATE_TESTS = ("mfma", "mfma_fma2", "mfma_fma3", "mfma_fma4", "mfma_fma6", "scan_tile", "xor_bcnt", "mfma_sign")


def bench_rates(args):
    """Instruction-rate tests (no memory traffic in the loops) on every CU,
    with one and two waves per SIMD: nanoseconds per unit per SIMD (an MFMA
    for the mfma* tests, a 16-token tile for scan_tile, a 128-bit (query row,
    token) Hamming pair for xor_bcnt and mfma_sign), and chip-wide rates."""
    import torch

    lib = ctypes.CDLL(os.path.join(ROOT, "maxsim_amd", "libmaxsim_rates.so"))
    lib.msim_rate_test.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.POINTER(ctypes.c_double)]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    iters = {"xor_bcnt": 4000, "mfma_sign": 4000, "scan_tile": 2000}
    out = {}
    for name in RATE_TESTS:
        row = {}
        for wps in (1, 2):
            ns = ctypes.c_double(0.0)
            if lib.msim_rate_test(name.encode(), cus, wps, iters.get(name, 4000), ctypes.byref(ns)) != 0:
                raise SystemExit(f"rate test {name} failed")
            row[f"ns_per_unit_{wps}w"] = ns.value
        simds = 4 * cus
        if name.startswith("mfma") and name != "mfma_sign":
            row["int8_tops_2w"] = 32768 * simds / row["ns_per_unit_2w"] / 1e3
        if name in ("xor_bcnt", "mfma_sign"):
            row["pairs_per_ns_chip_2w"] = simds / row["ns_per_unit_2w"]
        out[name] = row
        print(f"{name:10s} " + " ".join(f"{k}={v:.3f}" for k, v in row.items()), file=sys.stderr, flush=True)
    return {"metric": "instruction-rate tests", "cus": cus, "tests": out,
            "units": {"mfma*": "one v_mfma_i32_16x16x64_i8 (with its fmas)", "scan_tile": "one 16-token tile",
                      "xor_bcnt": "one 128-dim (query row, token) pair", "mfma_sign": "one 128-dim pair"},
            "metadata": host_metadata()}


def main():
    args = parse_args()
    if args.summarize_pmc:
        print(json.dumps(summarize_pmc(*args.summarize_pmc), indent=1))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported: this build "
              "scores on a single MI355X (documents would shard across GPUs with a top-k merge, not built here)",
              file=sys.stderr)
        sys.exit(2)
    if args.rates:
        print(json.dumps(bench_rates(args)), flush=True)
    elif args.pack:
        print(json.dumps(bench_pack(args)), flush=True)
    elif args.config == 2:
        bench_config2(args)
    else:
        print(json.dumps(OTHER_CONFIGS[args.config](args)), flush=True)


if __name__ == "__main__":
    main()
