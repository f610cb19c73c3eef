"""Benchmark of the nacho GPU path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2|c3]

A step is one call of the hot path over one batch of synthetic input, with the operands
already resident in HBM: `nacho_amd.gpu_csr_add_f32(A, B)` for the default workload (C2:
two 2^20 x 2^20 CSR matrices with rescaled Zipf(1.6) row lengths, 16.7M nonzeros each).
A call includes result allocation from the device pool, both kernels and the explicit
readback of the result length, exactly what a caller of the entry point waits for.  Steps
rotate over several independent copies of the operands so that no step re-reads inputs
still resident in the 256 MB Infinity Cache.

Prints ONE JSON line:
  value            whole-job throughput: algorithmic bytes per step / wall time per step
  roofline         the call's device pipeline (partition, count and write kernels, bracketed
                   by HIP events on the launch stream): algorithmic bytes per call / its
                   average duration, vs 8 TB/s;
                   `traffic` = measured HBM bytes per launch (rocprofv3 FETCH_SIZE +
                   WRITE_SIZE, calibrated on a copy kernel) when profiles/ holds them
  cpu_baseline     the C restatement of the reference's CPU kernel (oracle/) on this host's
                   cores over a bounded sample of the same workload
Algorithmic bytes (CSR add/mul) = 3*4*(rows+1) + 8*(nnzA + nnzB + nnzC).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

METRIC = ("effective HBM GB/s (% of MI355X peak) for csr_add/mul; ESC SpGEMM GFLOP/s")
PEAK_HBM_GBS = 8000.0
ROTATE = 4  # independent operand copies cycled through by the timed steps

WORKLOADS = {
    "c2": dict(op="add", kernel="csr_partition_kernel + csr_count_kernel<Union> + "
                              "csr_write_kernel<Union> (one call's device pipeline)",
               desc="C2 csr_add f32 2^20x2^20, Zipf(1.6) rows rescaled to mean 16 "
                    "(16.7M nnz each), seeds 1/2"),
    "c3": dict(op="mul", kernel="csr_partition_kernel + csr_count_kernel<Intersect> + "
                              "csr_write_kernel<Intersect> (one call's device pipeline)",
               desc="C3 csr_mul f32 2^20x2^20, A as C2, B = 50% of A + fresh columns "
                    "(seed 3)"),
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_operands(workload):
    from nacho_amd import synth

    if workload == "c2":
        return synth.c2_operands()
    return synth.c3_operands()


def traffic_from_profiles(workload):
    """Measured HBM bytes per launch of the dominant kernel, if profiled (else None)."""
    path = REPO / "profiles" / f"csr_merge_{workload}_traffic.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def cpu_baseline(workload, op, a, b, rows, bytes_per_call, budget_s):
    """Time the oracle's C restatement of the reference CPU kernel on this host."""
    from oracle import oracle

    cores = len(os.sched_getaffinity(0))
    cores = max(1, min(cores, 64))
    times = []
    start = time.perf_counter()
    while time.perf_counter() - start < budget_s and len(times) < 50:
        t = {}
        oracle.port_csr_binary(op, rows, *a, *b, nthreads=cores, timing=t)
        times.append(t["seconds"])
    times.sort()
    trimmed = times[1:-1] if len(times) > 4 else times
    sec = sum(trimmed) / len(trimmed)
    return {
        "value": round(bytes_per_call / sec / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{len(times)} full {workload} calls of the C restatement "
                  f"(oracle/nacho_oracle.c), mean of the middle {len(trimmed)}: "
                  f"{sec * 1e3:.1f} ms/call",
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="c2")
    ap.add_argument("--cpu-budget", type=float, default=12.0,
                    help="seconds of CPU baseline timing (0 disables)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 1 GiB device copy (rocprof counter calibration)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested).", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    device = torch.device("cuda:0")

    if args.calibrate_copy:
        n = 1 << 28  # 1 GiB of float32
        src = torch.ones(n, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read": 4 * n, "bytes_written": 4 * n,
                          "launches": 5}))
        return

    import nacho_amd
    from nacho_amd import synth

    spec = WORKLOADS[args.workload]
    t0 = time.perf_counter()
    a_np, b_np = make_operands(args.workload)
    rows = len(a_np[0]) - 1
    log(f"generated {args.workload}: rows={rows} nnzA={len(a_np[1])} nnzB={len(b_np[1])} "
        f"in {time.perf_counter() - t0:.1f}s")

    def upload(t):
        pos, crd, val = (torch.from_numpy(x).to(device) for x in t)
        return nacho_amd.CSR_gpu(pos, crd, val, torch.tensor([rows, rows], dtype=torch.int32))

    copies = [(upload(a_np), upload(b_np)) for _ in range(ROTATE)]
    fn = nacho_amd.gpu_csr_add_f32 if spec["op"] == "add" else nacho_amd.gpu_csr_mul_f32

    z = fn(*copies[0])
    torch.cuda.synchronize()
    nnz_c = int(z.dim_j_indices.numel())
    del z
    alg_bytes = synth.csr_bytes(rows, len(a_np[1]), len(b_np[1]), nnz_c)
    log(f"nnzC={nnz_c} algorithmic bytes/call={alg_bytes}")

    # warmup, then per-launch kernel durations (HIP events on the launch stream)
    nacho_amd.set_kernel_timing(True)
    for i in range(args.warmup):
        fn(*copies[i % ROTATE])
    torch.cuda.synchronize()
    kernel_ms = []
    for i in range(args.steps):
        fn(*copies[i % ROTATE])
        kernel_ms.append(nacho_amd.last_kernel_ms())
    nacho_amd.set_kernel_timing(False)
    torch.cuda.synchronize()

    # timed region: exactly K steps, synchronized on both sides
    torch.cuda.synchronize()
    start = time.perf_counter()
    for i in range(args.steps):
        fn(*copies[i % ROTATE])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    ms_per_step = elapsed * 1e3 / args.steps
    value = alg_bytes / (ms_per_step * 1e-3) / 1e9

    kernel_avg_ms = sum(kernel_ms) / len(kernel_ms)
    achieved = alg_bytes / (kernel_avg_ms * 1e-3) / 1e9
    log(f"kernel avg {kernel_avg_ms * 1e3:.1f} us -> {achieved:.0f} GB/s; "
        f"call {ms_per_step * 1e3:.1f} us -> {value:.0f} GB/s")

    cpu = None
    if args.cpu_budget > 0:
        cpu = cpu_baseline(args.workload, spec["op"], a_np, b_np, rows, alg_bytes,
                           args.cpu_budget)
        log(f"cpu baseline {cpu['value']} GB/s on {cpu['cores']} threads")

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded generators in nacho_amd/synth.py)",
        "config": {
            "workload": spec["desc"],
            "rows": rows,
            "nnz_a": len(a_np[1]),
            "nnz_b": len(b_np[1]),
            "nnz_c": nnz_c,
            "algorithmic_bytes_per_step": alg_bytes,
            "percent_of_peak_hbm": round(100.0 * value / PEAK_HBM_GBS, 2),
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": spec["kernel"],
            "achieved": round(achieved, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic_from_profiles(args.workload),
            "kernel_avg_us": round(kernel_avg_ms * 1e3, 2),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
