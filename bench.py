#!/usr/bin/env python3
"""Benchmark of the decode hot path on one MI355X.

Default workload: the Q4_K x Q8_K GEMV at 17408 x 5120 (the FFN gate/up shape
of the 27B model), quantised activations resident in HBM, weights rotated over
>= 1 GiB of distinct copies so every launch streams from HBM rather than the
256 MB last-level cache.  A "step" is one GEMV launch over one weight copy.

Prints one JSON line (see the fields below).  `roofline.achieved` is the
algorithmic bytes of one launch divided by its average duration measured
with HIP events on the stream the kernels run on.  `cpu_baseline` times the
reference's own AVX2 kernels (oracle/_ref, compiled from its sources) on
this host's cores over a bounded sample.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen3.8-27b-in-c_amd"))

PEAK_HBM_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--workload", default="q4k_gemv",
                   choices=["q4k_gemv", "q4k_gemv_t", "iq1m_gemv", "iq1m_gemv_t", "q6k_gemv"])
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    return p.parse_args()


WORKLOADS = {
    # name: (type, rows, width, label)
    "q4k_gemv": (12, 17408, 5120, "Q4_K GEMV 17408x5120"),
    "q4k_gemv_t": (12, 5120, 17408, "Q4_K GEMV 5120x17408"),
    "iq1m_gemv": (29, 17408, 5120, "IQ1_M GEMV 17408x5120"),
    "iq1m_gemv_t": (29, 5120, 17408, "IQ1_M GEMV 5120x17408"),
    "q6k_gemv": (14, 17408, 5120, "Q6_K GEMV 17408x5120"),
}
BLOCK = {12: 144, 14: 210, 29: 56}


def algorithmic_bytes(qtype, rows, width):
    """weights + Q8_K activation blocks + fp32 outputs of one GEMV launch"""
    return rows * (width // 256) * BLOCK[qtype] + (width // 256) * 292 + rows * 4


def cpu_baseline(qtype, rows, width, budget_s=12.0):
    """The reference's AVX2 GEMV (oracle/_ref) on the host cores, bounded sample."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Reference
    if not Reference.available():
        return None
    from q38hip import synth
    ref = Reference()
    w = synth.matrix(qtype, rows, width, seed=1)
    x = synth.activations(width, seed=2)
    q = ref.quantize(x.reshape(-1))
    ref.gemv(qtype, w, rows, q)  # warm-up
    times = []
    start = time.perf_counter()
    while time.perf_counter() - start < budget_s and len(times) < 400:
        t0 = time.perf_counter()
        ref.gemv(qtype, w, rows, q)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(algorithmic_bytes(qtype, rows, width) / med / 1e9, 3), "unit": "GB/s",
            "cores": threads, "kind": "reference",
            "sample": "median of %d single-row GEMVs (%s) over %.1f s, OpenMP threads=%d" % (
                len(times), WORKLOADS_LABEL[(qtype, rows, width)], time.perf_counter() - start, threads)}


WORKLOADS_LABEL = {(v[0], v[1], v[2]): v[3] for v in WORKLOADS.values()}


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import q38hip
    from q38hip import synth

    qtype, rows, width, label = WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    nbytes = algorithmic_bytes(qtype, rows, width)
    wbytes = rows * (width // 256) * BLOCK[qtype]
    copies = max(2, -(-(1 << 30) // wbytes) + 1)
    base = torch.from_numpy(synth.matrix(qtype, rows, width, seed=1)).to(dev)
    weights = [base] + [base.clone() for _ in range(copies - 1)]
    x = torch.from_numpy(synth.activations(width, seed=2)).to(dev)
    xq = q38hip.quantize_q8_k(x)
    out = torch.empty((1, rows), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream()

    for i in range(args.warmup):
        q38hip.gemm_q8_k(weights[i % copies], qtype, width, rows, xq, 1, out=out)
    torch.cuda.synchronize()

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(args.steps):
        q38hip.gemm_q8_k(weights[i % copies], qtype, width, rows, xq, 1, out=out)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # back-to-back launches on one stream: the event span / K is the average
    # launch duration including the inter-kernel gaps
    per_launch_ms = start.elapsed_time(end) / args.steps
    achieved = nbytes / (per_launch_ms * 1e-3) / 1e9

    result = {
        "metric": "quant-GEMV HBM GB/s (Q4_K x Q8_K decode GEMV)",
        "value": round(achieved, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xuint4->int32, fp32",
        "data": "synthetic (seeded GGUF blocks, N(0,1) activations)",
        "config": {"workload": label, "weight_copies_rotated": copies,
                   "rotated_bytes": copies * wbytes, "bytes_per_launch": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None},
        "cpu_baseline": None if args.no_cpu else cpu_baseline(qtype, rows, width),
    }
    print(json.dumps(result))


if __name__ == "__main__":
    main()
