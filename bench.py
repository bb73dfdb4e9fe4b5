#!/usr/bin/env python3
"""Benchmark of the decode hot path on one MI355X.

Default workload (`decode`): greedy decoding of the 27B-shaped Q4_K_M model
(64 layers, hidden 5120, FFN 17408, vocab 248320, Q6_K LM head, one MTP
block; random-init weights from the seeded synthetic GGUF writer) with MTP
draft length 3 through the engine ABI (q38_model_speculative_greedy): a
512-token random prompt is prefilled, then 256 tokens are decoded.  A "step"
is one speculative transaction; `value` is decoded tokens per second.
The `roofline` object is that of the dominant kernel of the step: the
matrix-core Q4_K x Q8_K GEMM over the 16-row tiled weights at the verify
batch's shape, 3 tokens x 34816 x 5120 (the fused FFN gate|up projection,
64 launches per transaction), timed in the same run on its own with the
weights rotated over >= 1 GiB of distinct copies.

`--layout iq1m` runs the same on the IQ1_M layout of the model (IQ1_M layer
matrices, Q4_K embedding, Q6_K LM head): a 4096-token prompt is prefilled
(`prefill_tokens_per_s`), then 1024 tokens are decoded (context 5124+); its
roofline is the IQ1_M GEMM of the fused FFN gate|up at 3 tokens.

Kernel workloads (`q4k_gemv`, `q4k_tiled_m3` ...): one GEMV / GEMM alone,
quantised activations resident in HBM, weights rotated over >= 1 GiB of
distinct copies so every launch streams from HBM rather than the 256 MB
last-level cache; a "step" is one launch.

Prints one JSON line (see the fields below).  `roofline.achieved` is the
algorithmic bytes of one launch divided by its average duration measured
with HIP events on the stream the kernels run on.  `roofline.traffic` is the
HBM bytes per launch read from the committed counter summary
profiles/<kernel>.<workload>.pmc.txt (rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated
against a plain device copy), or null when there is none.  `cpu_baseline`
times the reference's own AVX2 kernels (oracle/_ref, compiled from its
sources) on this host's cores over a bounded sample whose weights rotate over
more distinct copies than the host caches hold.

`--workload copy` times a plain device-to-device copy of 64 MiB buffers; it
is the calibration run for the memory counters, not a bench line.

`--trace-summary DIR` prints, from a rocprofv3 `--kernel-trace --output-format
csv` directory, the calls and average / min / max duration of every kernel
per launch grid (one kernel name serves several matrix shapes; the grid tells
them apart), and exits; `--trace-transactions N` restricts a decode run's
trace to its N transactions and reports each kernel's time per transaction.
"""
import argparse
import glob
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen3.8-27b-in-c_amd"))

PEAK_HBM_GBS = 8000.0

WORKLOADS = {
    # name: (type, rows, width, tokens, tiled, label)
    "q4k_gemv": (12, 17408, 5120, 1, True, "Q4_K GEMV 17408x5120"),
    "q4k_gemv_t": (12, 5120, 17408, 1, True, "Q4_K GEMV 5120x17408"),
    "iq1m_gemv": (29, 17408, 5120, 1, True, "IQ1_M GEMV 17408x5120"),
    "iq1m_gemv_t": (29, 5120, 17408, 1, True, "IQ1_M GEMV 5120x17408"),
    "q6k_gemv": (14, 17408, 5120, 1, False, "Q6_K GEMV 17408x5120"),
    "q6k_lmhead": (14, 248320, 5120, 1, False, "Q6_K LM head 248320x5120, one row (an MTP draft)"),
    "q6k_lmhead_m3": (14, 248320, 5120, 3, False, "Q6_K LM head 248320x5120, 3 rows (the verify batch)"),
    "q4k_tiled_m3": (12, 34816, 5120, 3, True, "Q4_K tiled GEMM 34816x5120 (FFN gate|up), 3 tokens"),
    "q4k_tiled_down_m3": (12, 5120, 17408, 3, True, "Q4_K tiled GEMM 5120x17408 (FFN down), 3 tokens"),
    "q4k_tiled_dnin_m3": (12, 16480, 5120, 3, True, "Q4_K tiled GEMM 16480x5120 (DeltaNet input group), 3 tokens"),
    "q4k_tiled_qkv_m3": (12, 14336, 5120, 3, True, "Q4_K tiled GEMM 14336x5120 (attention q|gate|k|v), 3 tokens"),
    "q4k_tiled_out_m3": (12, 5120, 6144, 3, True,
                         "Q4_K tiled GEMM 5120x6144 (attention output / DeltaNet output), 3 tokens"),
    "iq1m_gemm_m3": (29, 34816, 5120, 3, True, "IQ1_M GEMM 34816x5120 (FFN gate|up), 3 tokens"),
    "iq1m_gemm_down_m3": (29, 5120, 17408, 3, True, "IQ1_M GEMM 5120x17408 (FFN down), 3 tokens"),
    "iq1m_gemm_out_m3": (29, 5120, 6144, 3, True,
                         "IQ1_M GEMM 5120x6144 (attention output / DeltaNet output), 3 tokens"),
    "q4k_tiled_m8": (12, 34816, 5120, 8, True, "Q4_K tiled GEMM 34816x5120 (FFN gate|up), 8 tokens (prefill batch)"),
    "iq1m_gemm_m8": (29, 34816, 5120, 8, True, "IQ1_M GEMM 34816x5120 (FFN gate|up), 8 tokens (prefill batch)"),
    "q4k_wide_m256": (12, 34816, 5120, 256, True, "Q4_K tiled GEMM 34816x5120 (FFN gate|up), 256 tokens (prefill)"),
    "iq1m_wide_m256": (29, 34816, 5120, 256, False, "IQ1_M GEMM 34816x5120 (FFN gate|up), 256 tokens (prefill)"),
    "q4k_wide_down_m256": (12, 5120, 17408, 256, True, "Q4_K tiled GEMM 5120x17408 (FFN down), 256 tokens (prefill)"),
    "q4k_wide_m512": (12, 34816, 5120, 512, True, "Q4_K tiled GEMM 34816x5120 (FFN gate|up), 512 tokens (prefill)"),
    "iq1m_wide_m512": (29, 34816, 5120, 512, False, "IQ1_M GEMM 34816x5120 (FFN gate|up), 512 tokens (prefill)"),
    "q4k_wide_m4096": (12, 34816, 5120, 4096, True,
                       "Q4_K tiled GEMM 34816x5120 (FFN gate|up), 4096 tokens (one prefill batch)"),
    "iq1m_wide_m4096": (29, 34816, 5120, 4096, False,
                        "IQ1_M GEMM 34816x5120 (FFN gate|up), 4096 tokens (one prefill batch)"),
    "iq1m_wide_down_m4096": (29, 5120, 17408, 4096, False,
                             "IQ1_M GEMM 5120x17408 (FFN down), 4096 tokens (one prefill batch)"),
}
# device kernel each launch of a workload runs (q38hip dispatch for that shape; the
# trace summaries and counter profiles under profiles/ name the same kernels)
DEVICE_KERNEL = {
    "q4k_gemv": "gemv_q4k_lanes<20, 4, 1>",
    "q4k_gemv_t": "gemv_q4k_lanes<68, 12, 1>",
    "iq1m_gemv": "gemm_iq1m_dot4<20, 15, 2, 1>",
    "iq1m_gemv_t": "gemm_iq1m_dot4<68, 16, 2, 1>",
    "q4k_tiled_m3": "gemm_q4k_mm16<3, 20, 9, 4, 1>",
    "q4k_tiled_down_m3": "gemm_q4k_t32r<3, 68, 8, 1>",
    "q4k_tiled_out_m3": "gemm_q4k_t32r<3, 24, 8, 1>",
    "iq1m_gemm_m3": "gemm_iq1m_dot4<20, 15, 2, 3>",
    "iq1m_gemm_down_m3": "gemm_iq1m_dot4<68, 16, 2, 3>",
    "iq1m_gemm_out_m3": "gemm_iq1m_dot4<24, 12, 2, 3>",
}
# dense matrix-core peaks of MI355X, TOP/s: the Q4_K GEMM runs fp16 MFMA, IQ1_M int8
MFMA_PEAK_TOPS = {12: ("f16", 2500.0), 29: ("i8", 5000.0)}
BLOCK = {12: 144, 14: 210, 29: 56}
TYPE_NAME = {12: "Q4_K", 14: "Q6_K", 29: "IQ1_M"}
COPY_BYTES = 64 << 20


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None)
    p.add_argument("--warmup", type=int, default=None)
    p.add_argument("--workload", default="decode", choices=["decode", "prefill"] + sorted(WORKLOADS) + ["copy"])
    p.add_argument("--decode-tokens", type=int, default=None,
                   help="tokens decoded on every run (256 for q4km, 1024 for iq1m); --steps picks the timed window")
    p.add_argument("--layout", default="q4km", choices=["q4km", "iq1m"],
                   help="decode workload: Q4_K_M layout (default) or IQ1_M layer matrices")
    p.add_argument("--prompt", type=int, default=None, help="prompt tokens (512 for q4km, 4096 for iq1m)")
    p.add_argument("--draft", type=int, default=3)
    p.add_argument("--plain-tokens", type=int, default=32, help="plain greedy tokens after the timed region")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline time per thread count")
    p.add_argument("--no-extra", action="store_true",
                   help="decode: only the headline line (no verify block, IQ1_M or accepted-draft runs)")
    p.add_argument("--cpu-worker", action="store_true", help=argparse.SUPPRESS)
    p.add_argument("--cpu-gemv-worker", action="store_true", help=argparse.SUPPRESS)
    p.add_argument("--cpu-workloads", default="", help=argparse.SUPPRESS)
    p.add_argument("--cpu-calls", type=int, default=30, help=argparse.SUPPRESS)
    p.add_argument("--cpu-threads", default="", help=argparse.SUPPRESS)
    p.add_argument("--trace-summary", metavar="DIR", help="summarise a rocprofv3 kernel trace and exit")
    p.add_argument("--trace-transactions", type=int, default=0,
                   help="with --trace-summary of a decode run: its transaction count (warmup + steps)")
    return p.parse_args()


def algorithmic_bytes(qtype, rows, width, tokens=1):
    """weights + Q8_K activation blocks + fp32 outputs of one launch"""
    return rows * (width // 256) * BLOCK[qtype] + tokens * (width // 256) * 292 + tokens * rows * 4


def committed_traffic(workload):
    """HBM bytes per launch from profiles/<kernel>.<workload>.pmc.txt, or None."""
    paths = glob.glob(os.path.join(ROOT, "profiles", "*.%s.pmc.txt" % workload))
    if len(paths) != 1:
        return None
    with open(paths[0]) as f:
        m = re.search(r"^hbm_bytes_per_launch:\s*([0-9.]+)", f.read(), re.M)
    return float(m.group(1)) if m else None


def cpu_baseline(qtype, rows, width, tokens, budget_s):
    """The reference's AVX2 GEMV / GEMM (oracle/_ref) on the host cores,
    bounded sample.

    The weights rotate over enough distinct copies (>= 512 MB) that each call
    streams its matrix from DRAM as the GPU launches stream theirs from HBM."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Reference
    if not Reference.available():
        return None
    from q38hip import synth
    ref = Reference()
    base = synth.matrix(qtype, rows, width, seed=1)
    copies = max(2, -(-(512 << 20) // base.nbytes))
    weights = [base] + [base.copy() for _ in range(copies - 1)]
    x = synth.activations(width, seed=2, count=tokens)
    q = ref.quantize(x.reshape(-1))

    def call(w):
        if tokens == 1:
            ref.gemv(qtype, w, rows, q)
        else:
            ref.gemm(qtype, w, rows, q, tokens)

    call(weights[0])  # warm-up (thread pool start)
    count = 0
    start = time.perf_counter()
    while True:
        call(weights[count % copies])
        count += 1
        elapsed = time.perf_counter() - start
        if elapsed >= budget_s:
            break
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    entry = "q38_tensor_gemv_q8_k" if tokens == 1 else "q38_tensor_gemm_q8_k"
    return {"value": round(algorithmic_bytes(qtype, rows, width, tokens) * count / elapsed / 1e9, 3),
            "unit": "GB/s", "cores": threads, "kind": "reference",
            "sample": "%d %d-token %s x Q8_K products %dx%d (%s, AVX2 build), "
                      "weights rotated over %d copies (%d MB), %.1f s, OpenMP threads=%d" % (
                          count, tokens, TYPE_NAME[qtype], rows, width, entry, copies,
                          copies * base.nbytes >> 20, elapsed, threads)}


def timed(torch, stream, steps, launch):
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        launch(i)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # back-to-back launches on one stream: the event span / K is the average
    # launch duration including the inter-kernel gaps
    return start.elapsed_time(end) / steps, wall


def run_copy(torch, args):
    dev = torch.device("cuda:0")
    n = COPY_BYTES // 4
    bufs = [torch.empty(n, dtype=torch.float32, device=dev).fill_(i) for i in range(32)]
    stream = torch.cuda.current_stream()
    launch = lambda i: bufs[(2 * i + 1) % 32].copy_(bufs[(2 * i) % 32])  # noqa: E731
    steps = args.steps if args.steps is not None else 100
    for i in range(args.warmup if args.warmup is not None else 10):
        launch(i)
    per_ms, wall = timed(torch, stream, steps, launch)
    print(json.dumps({"metric": "device copy GB/s (counter calibration)", "value":
                      round(2 * COPY_BYTES / (per_ms * 1e-3) / 1e9, 2), "unit": "GB/s",
                      "bytes_read_per_launch": COPY_BYTES, "bytes_written_per_launch": COPY_BYTES,
                      "steps": steps, "ms_per_step": round(wall * 1e3 / steps, 5)}))


def kernel_roofline(torch, workload, steps, warmup):
    """Time `steps` back-to-back launches of one GEMV / GEMM workload on the
    current stream (HIP events); returns (per-launch ms, wall s, roofline
    dict, weight copies)."""
    import q38hip
    from q38hip import synth
    qtype, rows, width, tokens, tiled, label = WORKLOADS[workload]
    dev = torch.device("cuda:0")
    nbytes = algorithmic_bytes(qtype, rows, width, tokens)
    base = torch.from_numpy(synth.matrix(qtype, rows, width, seed=1)).to(dev)
    if tiled:
        # the engine's 16-row tiled copies (Q4_K, and IQ1_M for 1..8 tokens)
        base = (q38hip.repack_iq1m_tiles if qtype == 29 else q38hip.repack_q4k_tiles)(base, width, rows)
    copies = max(2, -(-(1 << 30) // base.numel()) + 1)
    # one allocation holds every copy, as the engine holds all weights in one
    pool = torch.empty(copies * base.numel(), dtype=torch.uint8, device=dev)
    weights = [pool[i * base.numel():(i + 1) * base.numel()] for i in range(copies)]
    for w in weights:
        w.copy_(base)
    x = torch.from_numpy(synth.activations(width, seed=2, count=tokens)).to(dev)
    xq = q38hip.quantize_q8_k(x.reshape(tokens, width))
    out = torch.empty((tokens, rows), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream()

    def launch(i):
        if tiled and qtype == 29:
            q38hip.gemm_q8_k_iq1m_tiled(weights[i % copies], width, rows, xq, tokens, out=out)
        elif tiled:
            q38hip.gemm_q8_k_tiled(weights[i % copies], width, rows, xq, tokens, out=out)
        else:
            q38hip.gemm_q8_k(weights[i % copies], qtype, width, rows, xq, tokens, out=out)

    for i in range(warmup):
        launch(i)
    per_launch_ms, wall = timed(torch, stream, steps, launch)
    achieved = nbytes / (per_launch_ms * 1e-3) / 1e9
    traffic = committed_traffic(workload)
    roofline = {"bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None if traffic is None else int(traffic),
                "kernel": "%s (%s)" % (DEVICE_KERNEL.get(workload, "gemm_q4k_tiled" if tiled else "gemm_q8k"), label),
                "bytes_per_launch": nbytes, "launch_us": round(per_launch_ms * 1e3, 3)}
    if (tiled and tokens > 1) or qtype == 29:
        # matrix-core kernels: algorithmic multiply-adds (2 ops each) per second
        kind, peak = MFMA_PEAK_TOPS[qtype]
        ops = 2 * rows * width * tokens
        tops = ops / (per_launch_ms * 1e-3) / 1e12
        roofline["matrix"] = {"mfma": kind, "ops_per_launch": ops, "achieved": round(tops, 3), "peak": peak,
                              "unit": "TOP/s", "frac": round(tops / peak, 5)}
    del weights, pool, base
    return per_launch_ms, wall, roofline, copies


def _trace_rows(directory):
    import csv
    paths = glob.glob(os.path.join(directory, "**", "*kernel_trace.csv"), recursive=True)
    if not paths:
        raise SystemExit("no *kernel_trace.csv under %s" % directory)
    rows = []
    for path in paths:
        with open(path) as f:
            rows.extend(csv.DictReader(f))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    for r in rows:
        name = r["Kernel_Name"].replace("void ", "").replace("q38::", "").replace("(anonymous namespace)::", "")
        r["short"] = re.sub(r"\(.*$", "", name)
        r["groups"] = int(r["Grid_Size_X"]) // max(int(r["Workgroup_Size_X"]), 1)
        r["ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    return rows


def trace_summary(directory, transactions=0):
    """calls / avg / min / max ns per (kernel, grid) of a rocprofv3 kernel
    trace.  With `transactions` > 0 the trace is that of the decode workload
    and only its transactions are summarised: the dispatches after the
    prefill's last GEMM (a prompt-batch or 8-token Q4_K / IQ1_M GEMM) and before the first
    kernel of the roofline run that follows (its weight repack or its
    activation quantisation, which the model never launches), reported per
    transaction."""
    rows = _trace_rows(directory)
    if transactions:
        names = [r["short"] for r in rows]
        prefill = ("gemm_q4k_wide", "gemm_iq1m_wide", "gemm_q4k_tiled<8", "gemm_q4k_t32<8", "gemm_iq1m_mfma<8")
        first = max(i for i, n in enumerate(names) if n.startswith(prefill)) + 1
        # the decode ends with the last transaction's verify tail (the
        # roofline runs that follow launch none); the wall clock stops there
        last = max(i for i, n in enumerate(names) if n.startswith(("accept_kernel", "verify_tail_kernel"))) + 1
        rows = rows[first:last]
        wall =int(rows[-1]["End_Timestamp"]) - int(rows[0]["Start_Timestamp"])
        busy = sum(r["ns"] for r in rows)
        print("%d dispatches over %d transactions: %.3f ms wall and %.3f ms kernel time per transaction"
              % (len(rows), transactions, wall / 1e6 / transactions, busy / 1e6 / transactions))
    stats = {}
    for r in rows:
        s = stats.setdefault((r["short"], r["groups"], int(r["Workgroup_Size_X"])), [0, 0, r["ns"], r["ns"]])
        s[0] += 1
        s[1] += r["ns"]
        s[2] = min(s[2], r["ns"])
        s[3] = max(s[3], r["ns"])
    total = sum(v[1] for v in stats.values())
    per = " per_txn us/txn" if transactions else ""
    print("%-40s %7s %7s %7s %10s %8s %8s %6s%s" % ("kernel", "groups", "threads", "calls", "avg_ns", "min_ns",
                                                    "max_ns", "share", per))
    for (name, groups, threads), (calls, dsum, dmin, dmax) in sorted(stats.items(), key=lambda kv: -kv[1][1]):
        extra = " %7.2f %6.1f" % (calls / transactions, dsum / transactions / 1e3) if transactions else ""
        print("%-40s %7d %7d %7d %10.1f %8d %8d %5.1f%%%s" % (name[:40], groups, threads, calls, dsum / calls, dmin,
                                                             dmax, 100.0 * dsum / total, extra))


def prompt_ids(count, seed=11):
    return np.random.Generator(np.random.PCG64(seed)).integers(0, 248320, count).astype(np.uint32)


def host_cpu_info():
    """lscpu model name, physical cores (cores per socket x sockets), logical
    CPUs, and the C library version of this host."""
    import platform
    import subprocess
    info = {"model": platform.processor() or None, "physical_cores": None, "logical_cpus": os.cpu_count(),
            "glibc": "-".join(platform.libc_ver())}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, check=True).stdout
        fields = dict(line.split(":", 1) for line in out.splitlines() if ":" in line)
        fields = {k.strip(): v.strip() for k, v in fields.items()}
        info["model"] = fields.get("Model name", info["model"])
        info["physical_cores"] = int(fields["Core(s) per socket"]) * int(fields.get("Socket(s)", "1"))
    except (OSError, subprocess.CalledProcessError, KeyError, ValueError):
        pass
    # the CPU share this process may use (a container or job limit)
    try:
        info["usable_cpus"] = len(os.sched_getaffinity(0))
    except AttributeError:
        info["usable_cpus"] = os.cpu_count()
    return info


def cpu_decode_worker(args):
    """Child process of the CPU baseline (no GPU use): the reference engine
    (oracle/_ref, its own C sources, AVX2 + OpenMP build) prefills the same
    prompt as the GPU run, then runs speculative_greedy(draft) transactions
    for about `--cpu-seconds` at each thread count of --cpu-threads (OpenMP
    threads bound to cores).  Prints one JSON line."""
    import ctypes
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import reference_model
    from q38hip import synth
    path = synth.model_path(1, args.layout)
    threads = [int(t) for t in args.cpu_threads.split(",")]
    gomp = ctypes.CDLL("libgomp.so.1")
    gomp.omp_set_num_threads(threads[0])
    model = reference_model().open(path, args.prompt + 64 * args.draft + 16)
    model.enable_mtp()
    t0 = time.perf_counter()
    logits = model.prefill(prompt_ids(args.prompt))
    prefill_s = time.perf_counter() - t0
    token = int(np.argmax(logits))
    runs = []
    for n in threads:
        gomp.omp_set_num_threads(n)
        produced = transactions = 0
        start = time.perf_counter()
        while time.perf_counter() - start < args.cpu_seconds:
            accepted, _ = model.speculative_greedy(token, 0xFFFFFFFF, args.draft)
            produced += len(accepted)
            token = int(accepted[-1])
            transactions += 1
        elapsed = time.perf_counter() - start
        runs.append({"threads": n, "tokens": produced, "transactions": transactions, "seconds": round(elapsed, 2),
                     "tokens_per_s": round(produced / elapsed, 4)})
    model.close()
    print(json.dumps({"prefill_s": round(prefill_s, 2), "runs": runs}))


def cpu_gemv_worker(args):
    """Child process of the GEMV baselines (no GPU use): the reference's
    q38_quantize_q8_k + q38_tensor_gemv_q8_k (oracle/_ref, AVX2 + OpenMP
    build of src/qwen38/qwen38_quant.c) on the GEMV workloads of
    --cpu-workloads, each call timed on its own: warm-up, then the median of
    --cpu-calls calls at each thread count of --cpu-threads.  The weights
    rotate over >= 2 GB of copies so every call streams from DRAM.  Prints
    one JSON line."""
    import ctypes
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Reference
    from q38hip import synth
    ref = Reference()
    gomp = ctypes.CDLL("libgomp.so.1")
    threads = [int(t) for t in args.cpu_threads.split(",")]
    out = {}
    for workload in args.cpu_workloads.split(","):
        qtype, rows, width, tokens, _, label = WORKLOADS[workload]
        base = synth.matrix(qtype, rows, width, seed=1)
        copies = max(2, -(-(2 << 30) // base.nbytes))
        weights = [base] + [base.copy() for _ in range(copies - 1)]
        x = synth.activations(width, seed=2).reshape(-1)
        runs = []
        for n in threads:
            gomp.omp_set_num_threads(n)
            for i in range(3):
                ref.gemv(qtype, weights[i % copies], rows, ref.quantize(x))
            times = []
            for i in range(args.cpu_calls):
                t0 = time.perf_counter()
                ref.gemv(qtype, weights[i % copies], rows, ref.quantize(x))
                times.append(time.perf_counter() - t0)
            med = float(np.median(times))
            runs.append({"threads": n, "median_us": round(med * 1e6, 1), "calls": len(times),
                         "GB_s": round(algorithmic_bytes(qtype, rows, width) / med / 1e9, 3)})
        out[workload] = {"runs": runs, "copies": copies, "label": label}
    print(json.dumps(out))


def cpu_threads_plan():
    """(host info, thread counts): all physical cores of this process's CPU
    share, and 12 (the reference CLI's default, src/cli/qwen38_main.c:
    1431-1432) when different"""
    info = host_cpu_info()
    cores = min(info["physical_cores"] or info["usable_cpus"], info["usable_cpus"])
    return info, [cores] + ([12] if cores != 12 else [])


def cpu_gemv_baselines(workloads, calls=30):
    """The reference GEMV on the host cores for each workload (child process,
    OpenMP threads bound to cores); {workload: cpu_baseline object}."""
    import subprocess
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Reference
    if not Reference.available():
        return {}
    info, threads = cpu_threads_plan()
    env = dict(os.environ, OMP_NUM_THREADS=str(threads[0]), OMP_PROC_BIND="close", OMP_PLACES="cores")
    cmd = [sys.executable, os.path.abspath(__file__), "--cpu-gemv-worker", "--cpu-workloads", ",".join(workloads),
           "--cpu-calls", str(calls), "--cpu-threads", ",".join(str(t) for t in threads)]
    out = subprocess.run(cmd, env=env, capture_output=True, text=True)
    if out.returncode != 0:
        return {w: {"value": None, "error": out.stderr[-400:]} for w in workloads}
    res = json.loads(out.stdout.strip().splitlines()[-1])
    result = {}
    for w, r in res.items():
        main = r["runs"][0]
        result[w] = {"value": main["GB_s"], "unit": "GB/s", "cores": main["threads"], "kind": "reference",
                     "median_us": main["median_us"],
                     "sample": "median of %d calls of q38_quantize_q8_k + q38_tensor_gemv_q8_k (AVX2 + OpenMP build "
                               "of the reference's own sources), %s, weights rotated over %d copies, after 3 "
                               "warm-up calls, per thread count" % (main["calls"], r["label"], r["copies"]),
                     "runs": r["runs"], "host": info}
    return result


def cpu_decode_baseline(args, label="Q4_K_M", layout=None, prompt=None, seconds=None):
    """The reference engine on the host cores, run in a child process (it
    never touches the GPU) on the same GGUF as the GPU run: one sample on all
    physical cores (OMP_PROC_BIND=close, OMP_PLACES=cores), one at 12
    threads, the reference CLI's default (src/cli/qwen38_main.c:
    1431-1432)."""
    import subprocess
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Reference
    if not Reference.available():
        return None
    layout = layout or args.layout
    prompt = prompt or args.prompt
    seconds = seconds or args.cpu_seconds
    info, threads = cpu_threads_plan()
    env = dict(os.environ, OMP_NUM_THREADS=str(threads[0]), OMP_PROC_BIND="close", OMP_PLACES="cores")
    cmd = [sys.executable, os.path.abspath(__file__), "--cpu-worker", "--layout", layout,
           "--prompt", str(prompt), "--draft", str(args.draft), "--cpu-seconds", str(seconds),
           "--cpu-threads", ",".join(str(t) for t in threads)]
    out = subprocess.run(cmd, env=env, capture_output=True, text=True)
    if out.returncode != 0:
        return {"value": None, "error": out.stderr[-400:]}
    res = json.loads(out.stdout.strip().splitlines()[-1])
    main = res["runs"][0]
    return {"value": main["tokens_per_s"], "unit": "tokens/s", "cores": main["threads"], "kind": "reference",
            "sample": "reference engine (AVX2 + OpenMP build of its own sources) on the same synthetic 27B %s "
                      "GGUF and a %d-token prompt (prefill %.1f s), then q38_model_speculative_greedy(k=%d) "
                      "transactions for %.0f s per thread count" % (label, prompt, res["prefill_s"], args.draft,
                                                                      seconds),
            "runs": res["runs"], "prefill_s": res["prefill_s"],
            "prefill_tokens_per_s": round(prompt / res["prefill_s"], 2) if res["prefill_s"] else None,
            "host": info}


LAYOUTS = {
    # layout: (matrix types, dominant kernel workload, default prompt, default decoded tokens)
    "q4km": ("Q4_K_M", "q4k_tiled_m3", 512, 256),
    "iq1m": ("IQ1_M", "iq1m_gemm_m3", 4096, 1024),
}
# single-row GEMV rooflines reported beside the decode line, both shapes
GEMV_ROOFLINES = ("q4k_gemv", "q4k_gemv_t", "iq1m_gemv", "iq1m_gemv_t")
# the verify block: layer 3 (the first full-attention block) over a 2048-token cache
VERIFY_LAYER, VERIFY_CACHE, VERIFY_ROWS = 3, 2048, (1, 2, 3, 4, 5)
# Q4_K bytes of one full-attention block: q+gate 12288 rows, k and v 1024 rows
# (20 blocks each), output 5120 x 24 blocks, gate|up 34816 x 20, down 5120 x 68
BLOCK_WEIGHT_BYTES = 144 * (14336 * 20 + 5120 * 24 + 34816 * 20 + 5120 * 68)


def decode_fixture(layout):
    """Token ids the reference engine produced for this workload
    (tests/golden/decode_<layout>_s1.npz), or None."""
    path = os.path.join(ROOT, "tests", "golden", "decode_%s_s1.npz" % layout)
    if not os.path.exists(path):
        return None
    g = np.load(path)
    return [int(t) for t in g["spec_tokens"]] if int(g["prompt_len"][0]) else None


def decode_measure(torch, variant, prompt_len, decode_tokens, draft, warmup=8, window=None, plain_tokens=0,
                   mtp_variant=None, fixture=None):
    """Open the synthetic `variant` model (and the separate MTP checkpoint
    `mtp_variant`, if any), prefill `prompt_len` random ids, then decode
    through q38_model_speculative_greedy(k=draft) until `decode_tokens` are
    produced (or warmup + window transactions ran), timing the transactions
    after the first `warmup`; then `plain_tokens` plain greedy steps."""
    from q38hip import synth
    from q38hip.model import Model
    path = synth.model_path(1, variant)
    if path is None:
        raise SystemExit("no directory with room for the synthetic model (set Q38_MODEL_DIR)")
    t0 = time.perf_counter()
    synth.write_model_gguf(path, 1, variant)
    mtp_path = None
    if mtp_variant:
        mtp_path = synth.write_model_gguf(synth.model_path(1, mtp_variant), 1, mtp_variant)
    t_synth = time.perf_counter() - t0
    context = prompt_len + max(decode_tokens, (warmup + (window or 0)) * draft) + 4 * draft + plain_tokens + 16
    t0 = time.perf_counter()
    model = Model.open(path, context)
    if mtp_path:
        model.attach_mtp(mtp_path)
    t_open = time.perf_counter() - t0
    model.enable_mtp()
    prompt = prompt_ids(prompt_len)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits = model.prefill(prompt)
    t_prefill = time.perf_counter() - t0
    sequence = [int(np.argmax(logits))]
    counts = []
    t_start = t_end = None
    done = 0
    while len(sequence) < decode_tokens or (window is not None and done < warmup + window):
        if done == warmup:
            torch.cuda.synchronize()
            t_start = time.perf_counter()
        accepted, _ = model.speculative_greedy(sequence[-1], 0xFFFFFFFF, draft, logits=False)
        sequence.extend(int(t) for t in accepted)
        done += 1
        if done > warmup:
            counts.append(len(accepted))
        if window is not None and done == warmup + window:
            torch.cuda.synchronize()
            t_end = time.perf_counter()
    if t_end is None:
        torch.cuda.synchronize()
        t_end = time.perf_counter()
    if t_start is None:
        raise SystemExit("the warm-up (%d transactions) covers the whole decode" % warmup)
    wall = t_end - t_start
    steps = len(counts) if window is None else window
    produced = sum(counts[:steps])
    n = min(len(fixture), len(sequence)) if fixture else 0
    parity = (sequence[:n] == fixture[:n]) if fixture else None
    token = sequence[-1]
    t1 = time.perf_counter()
    for _ in range(plain_tokens):
        token = int(np.argmax(model.forward_token(token)))
    plain_wall = time.perf_counter() - t1
    model.close()
    return {"tokens_per_s": round(produced / wall, 3), "ms_per_step": round(wall * 1e3 / steps, 4), "steps": steps,
            "warmup": warmup, "prompt_tokens": prompt_len, "context": context,
            "decoded_tokens": len(sequence) - 1, "transactions": done, "timed_transactions": steps,
            "timed_tokens": produced, "accepted_per_transaction": round(produced / steps, 4),
            "token_parity_with_reference": parity, "token_parity_checked": n,
            "prefill_s": round(t_prefill, 3), "prefill_tokens_per_s": round(prompt_len / t_prefill, 1),
            "open_upload_s": round(t_open, 3), "synth_s": round(t_synth, 3),
            "plain_greedy_tokens_per_s": round(plain_tokens / plain_wall, 3) if plain_tokens else None}


def committed_mfma(workload):
    """MFMA busy fraction of a workload's kernel from the committed counter
    summary profiles/mfma_util.*.pmc.txt (a line 'mfma_busy <workload>: F'),
    or None"""
    for path in glob.glob(os.path.join(ROOT, "profiles", "mfma_util.*.pmc.txt")):
        with open(path) as f:
            m = re.search(r"^mfma_busy %s:\s*([0-9.]+)" % re.escape(workload), f.read(), re.M)
        if m:
            return float(m.group(1))
    return None


def verify_block_measure(torch):
    """cfg3: one full-attention block of the Q4_K_M model over `rows` verify
    rows at a 2048-token cache, as the speculative verify runs it, and the
    verify tail (argmax of the rows' logits, acceptance, row gather);
    device times from q38hip_model_time_block."""
    import ctypes
    from q38hip import synth
    from q38hip.model import Model
    path = synth.write_model_gguf(synth.model_path(1, "q4km"), 1, "q4km")
    model = Model.open(path, VERIFY_CACHE + 64)
    model.enable_mtp()
    lib = model.lib
    lib.q38hip_model_time_block.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                            ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)]
    model.prefill(prompt_ids(VERIFY_CACHE, seed=3))
    rows_out = {}
    for rows in VERIFY_ROWS:
        b, t = ctypes.c_float(), ctypes.c_float()
        if not lib.q38hip_model_time_block(model.handle, VERIFY_LAYER, rows, 200, ctypes.byref(b), ctypes.byref(t)):
            raise SystemExit("q38hip_model_time_block failed")
        # weights + K and V of every cached position (fp32) + Q8_K inputs and fp32 outputs of the projections
        kv = (VERIFY_CACHE + rows) * 1024 * 4 * 2
        act = rows * ((20 + 24 + 20 + 68) * 292 + (14336 + 5120 + 34816 + 5120) * 4)
        nbytes = BLOCK_WEIGHT_BYTES + kv + act
        rows_out[str(rows)] = {"block_us": round(b.value, 2), "tail_us": round(t.value, 2), "bytes": nbytes,
                               "achieved_GB_s": round(nbytes / (b.value * 1e-6) / 1e9, 1),
                               "frac": round(nbytes / (b.value * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}
    model.close()
    return {"workload": "one full-attention block (layer %d) of the 27B Q4_K_M model over k+1 verify rows at a "
                        "%d-token cache, then the verify tail (argmax of the rows' 248320 logits, greedy "
                        "acceptance, logits row gather); each a captured graph replayed 200 times "
                        "(q38hip_model_time_block)" % (VERIFY_LAYER, VERIFY_CACHE),
            "weights_bytes": BLOCK_WEIGHT_BYTES, "time_at_peak_us": round(BLOCK_WEIGHT_BYTES / PEAK_HBM_GBS / 1e3, 2),
            "rows": rows_out,
            "gate_up_mfma_busy": committed_mfma("q4k_tiled_m3")}


def run_prefill(torch, args):
    """The prompt evaluation alone (q38_model_prefill): the layout's model,
    its default prompt, one untimed call (module loads, first-use
    allocations), a reset, then one timed call.  Prints one JSON line."""
    from q38hip import synth
    from q38hip.model import Model
    label, _, default_prompt, _ = LAYOUTS[args.layout]
    prompt_len = args.prompt or default_prompt
    path = synth.write_model_gguf(synth.model_path(1, args.layout), 1, args.layout)
    model = Model.open(path, prompt_len + 16)
    model.enable_mtp()
    prompt = prompt_ids(prompt_len)
    model.prefill(prompt)
    model.reset()
    model.enable_mtp()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    model.prefill(prompt)
    wall = time.perf_counter() - t0
    model.close()
    print(json.dumps({"metric": "prefill tokens/s (27B %s, MTP catch-up included)" % label,
                      "value": round(prompt_len / wall, 1), "unit": "tokens/s", "n_gpus": 1, "steps": 1,
                      "warmup": 1, "ms_per_step": round(wall * 1e3, 3), "higher_is_better": True,
                      "config": {"workload": "prefill of a %d-token random prompt" % prompt_len}}))


def run_decode(torch, args):
    label, roof_workload, default_prompt, default_tokens = LAYOUTS[args.layout]
    if args.prompt is None:
        args.prompt = default_prompt
    decode_tokens = args.decode_tokens if args.decode_tokens is not None else default_tokens
    warmup = args.warmup if args.warmup is not None else 8
    d = decode_measure(torch, args.layout, args.prompt, decode_tokens, args.draft, warmup, args.steps,
                       args.plain_tokens, fixture=decode_fixture(args.layout))
    _, _, roofline, copies = kernel_roofline(torch, roof_workload, 200, 20)
    gemv = {}
    for workload in GEMV_ROOFLINES:
        _, _, r, _ = kernel_roofline(torch, workload, 200, 20)
        gemv[workload] = {k: r[k] for k in ("kernel", "achieved", "frac", "launch_us", "bytes_per_launch",
                                            "traffic")}
    config = {"workload": "decode 27B %s + MTP k=%d" % (label, args.draft), "layers": 64, "hidden": 5120,
              "ffn": 17408, "vocab": 248320}
    config.update({k: d[k] for k in ("prompt_tokens", "context", "decoded_tokens", "transactions",
                                     "timed_transactions", "timed_tokens", "accepted_per_transaction",
                                     "token_parity_with_reference", "token_parity_checked", "prefill_s",
                                     "prefill_tokens_per_s", "open_upload_s", "synth_s",
                                     "plain_greedy_tokens_per_s")})
    result = {
        "metric": "decode tokens/s (27B %s + MTP k=%d, greedy)" % (label, args.draft),
        "value": d["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": d["steps"],
        "warmup": warmup,
        "ms_per_step": d["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8x%s/Q6_K->i32, f32" % ("Q4_K" if args.layout == "q4km" else "IQ1_M"),
        "data": "synthetic (seeded random-init 27B %s GGUF, random prompt ids)" % label,
        "config": config,
        "roofline": roofline,
        "gemv_rooflines": gemv,
        "cpu_baseline": None if args.no_cpu else cpu_decode_baseline(args, label),
    }
    if args.layout == "q4km" and not args.no_extra:
        # the other configurations of the path, measured in the same run
        if not args.no_cpu:
            for w, b in cpu_gemv_baselines(GEMV_ROOFLINES).items():
                gemv[w]["cpu_baseline"] = b
        result["verify_block"] = verify_block_measure(torch)
        c5 = decode_measure(torch, "iq1m", 4096, 1024, args.draft, warmup=8, fixture=decode_fixture("iq1m"))
        c5["workload"] = ("27B IQ1_M layout (IQ1_M layer matrices, Q4_K embedding, Q6_K LM head): a 4096-token "
                          "prompt prefilled as one 4096-token batch on the matrix cores, then 1024 tokens decoded with "
                          "MTP k=%d (context 4097-5120)" % args.draft)
        c5["prefill_mfma_busy"] = {w: committed_mfma(w) for w in ("iq1m_wide_m4096", "iq1m_wide_m512",
                                                                   "q4k_wide_m512")}
        c5["cpu_baseline"] = None if args.no_cpu else cpu_decode_baseline(args, "IQ1_M", layout="iq1m", prompt=128,
                                                                           seconds=10.0)
        result["iq1m_prefill_decode"] = c5
        acc = {}
        for name, variant, mtp in (("all_drafts_accepted", "accept_all", None),
                                   ("accept_pair", "accept", "accept_mtp")):
            a = decode_measure(torch, variant, 512, 96, args.draft, warmup=4, mtp_variant=mtp)
            acc[name] = {k: a[k] for k in ("tokens_per_s", "ms_per_step", "timed_transactions", "timed_tokens",
                                           "accepted_per_transaction", "prefill_tokens_per_s")}
        acc["note"] = ("all_drafts_accepted: the Q4_K_M model with every LM head row equal, so every draft is "
                       "accepted; accept_pair: the 64-block model with a two-row LM head and its separate MTP "
                       "checkpoint, where about a third of the drafts are accepted; 512-token prompt, k=%d"
                       % args.draft)
        result["accepted_drafts"] = acc
    print(json.dumps(result))


def main():
    args = parse()
    if args.trace_summary:
        trace_summary(args.trace_summary, args.trace_transactions)
        return
    if args.cpu_worker:
        cpu_decode_worker(args)
        return
    if args.cpu_gemv_worker:
        cpu_gemv_worker(args)
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: the library has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if args.workload == "copy":
        run_copy(torch, args)
        return
    if args.workload == "decode":
        run_decode(torch, args)
        return
    if args.workload == "prefill":
        run_prefill(torch, args)
        return
    qtype, rows, width, tokens, tiled, label = WORKLOADS[args.workload]
    steps = args.steps if args.steps is not None else 200
    warmup = args.warmup if args.warmup is not None else 20
    per_launch_ms, wall, roofline, copies = kernel_roofline(torch, args.workload, steps, warmup)
    result = {
        "metric": "quant-%s HBM GB/s (%s x Q8_K, %d token%s)" % ("GEMV" if tokens == 1 else "GEMM",
                                                               TYPE_NAME[qtype], tokens, "s" if tokens > 1 else ""),
        "value": roofline["achieved"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(wall * 1e3 / steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8x%s->i32, f32" % TYPE_NAME[qtype],
        "data": "synthetic (seeded GGUF blocks, N(0,1) activations)",
        "config": {"workload": label, "weight_copies_rotated": copies,
                   "rotated_bytes": copies * rows * (width // 256) * BLOCK[qtype],
                   "bytes_per_launch": algorithmic_bytes(qtype, rows, width, tokens)},
        "roofline": roofline,
        "cpu_baseline": None if args.no_cpu else cpu_baseline(qtype, rows, width, tokens, args.cpu_seconds),
    }
    print(json.dumps(result))


if __name__ == "__main__":
    main()
