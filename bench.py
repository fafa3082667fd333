"""Benchmark of the MaxSim hot path on one MI355X.

One step = one pass of the hot path over one batch, device-resident and
enqueued on one stream (msim_int4_topk_int8q_async): int8 quantisation of the
fp32 query [4, 32, 128] (quantize_query_int8_kernel), the int4 x int8 MFMA
MaxSim scan over the whole per-token int4 corpus (4,096 docs, 64-192 tokens
each, dim 128; int8q_scan_kernel) and the device top-10 (topk_small_kernel).
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
import csv
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
SCAN_KERNEL = "int8q_scan_kernel"
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "int8q_scan_config2_traffic.md")
CALIBRATION_BYTES = 256 << 20  # one plain copy: reads and writes this many bytes
SCAN_BLOCK = 10  # scan launches between two events


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
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print HBM traffic per scan launch from two rocprofv3 --pmc runs and exit")
    return ap.parse_args()


def algorithmic_bytes(num_tokens: int, num_docs: int, batch: int, query_tokens: int) -> dict:
    """Bytes the scan kernel must move per launch over a per-token int4 corpus:
    64 B of int4 codes + 4 B token scale per token, 8 B per document offset,
    the quantised query (128 B codes + 4 B scale per query row, read once per
    workgroup from L2 but counted once) and the f32 score row per document."""
    corpus = 68 * num_tokens + 8 * (num_docs + 1)
    query = batch * query_tokens * (128 + 4)
    out = 4 * batch * num_docs
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


def cpu_baseline(packed, query, seconds: float):
    """The C oracle (one thread) on a bounded sample of the same workload: whole
    config-2 calls (quantise + scan of every document + top-10), repeated until
    about `seconds` have passed."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc

    orc.build()
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
    return {
        "value": docs / elapsed,
        "unit": "docs scored/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{reps} full config-2 call(s): [{query.shape[0]},{query.shape[1]},128] query x "
                  f"{packed.doc_offsets.shape[0] - 1} docs + top-10, C oracle (oracle/maxsim_oracle.c), "
                  f"1 thread, {elapsed:.1f} s",
        "ms_per_call": 1e3 * elapsed / reps,
    }


def main():
    args = parse_args()
    if args.summarize_pmc:
        print(json.dumps(summarize_pmc(*args.summarize_pmc), indent=1))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported: this build "
              "scores on a single MI355X (the sharding design is written up in DESIGN.md)",
              file=sys.stderr)
        sys.exit(2)

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
        # quantize_query_int8_kernel -> int8q_scan_kernel -> topk_small_kernel
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

    # ---- scan kernel alone: quantise once outside the events, then blocks of
    # SCAN_BLOCK back-to-back scan launches between two events on the launch
    # stream (consecutive launches on one stream start as the previous one
    # ends, so a block's time over SCAN_BLOCK is the kernel's duration).
    check(lib.msim_int4_quantize_int8q_async(handle._h, ptr(query), batch, qtok, sptr))
    blocks = max(1, args.steps // SCAN_BLOCK)
    sev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(blocks)]
    for i in range(blocks):
        sev[i][0].record(stream)
        for _ in range(SCAN_BLOCK):
            check(lib.msim_int4_score_int8q_async(handle._h, batch, qtok, ptr(scores), sptr))
        sev[i][1].record(stream)
    torch.cuda.synchronize()
    scan_ms = np.array([e[0].elapsed_time(e[1]) for e in sev]) / SCAN_BLOCK
    assert np.array_equal(scores.cpu().numpy(), ref_scores), "scan scores differ between entry points"

    nbytes = algorithmic_bytes(num_tokens, num_docs, batch, qtok)
    scan_avg_s = float(scan_ms.mean()) * 1e-3
    achieved = nbytes["total"] / scan_avg_s / 1e9

    # ---- MALL-cold: rotate over corpus copies whose total exceeds the 256 MB cache.
    cold = None
    if args.cold_copies > 0:
        copies = [handle] + [int4_to_device(packed).data for _ in range(args.cold_copies - 1)]
        for c in copies:
            step(c)
        torch.cuda.synchronize()
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

    # ---- synchronous host API (numpy in, numpy out), the reference's protocol.
    for _ in range(5):
        handle.topk_batch_int8q(query_np, k)
    api = []
    for _ in range(60):
        a = time.perf_counter()
        handle.topk_batch_int8q(query_np, k)
        api.append(1e3 * (time.perf_counter() - a))
    api = np.array(api)

    cpu = None if args.no_cpu_baseline else cpu_baseline(packed, query_np, args.cpu_seconds)
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
            "step": "quantize_query_int8_kernel + int8q_scan_kernel + topk_small_kernel on one stream, "
                    "device-resident (msim_int4_topk_int8q_async)",
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
            "note": "scan launches back to back, averaged over blocks of %d; the 35.7 MB corpus stays in the 256 MB MALL between launches" % SCAN_BLOCK,
        },
        "mall_cold": cold,
        "api_sync_ms": {"p50": float(np.percentile(api, 50)), "p95": float(np.percentile(api, 95))},
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
