"""Benchmark of the nacho GPU path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only]
                    [--workload c2|c3|c4|c5|c5coo|c2coo|c3coo|c2dcsr|c3dcsr|c2add3|c4sssmm
                                |c5inner|c5innercoo|c2coocsr]
    python bench.py --workload mtx --files A.mtx B.mtx [...]      (real data, local files)
    python bench.py --workload tns --files T.tns [...] [--dims I,J,K]

The default run prints the C2 csr_add line (the headline `value`) with a `workloads` list
holding the other north-star configurations measured in the same run: C3 csr_mul, C5
csf_add and coo3d_add, and C4 ESC SpGEMM (each with its call time, roofline and CPU
baseline).  `--only` (or any --workload other than c2) prints one workload's line alone.

A step is one call of the hot path over one batch of synthetic input, with the operands
already resident in HBM: `nacho_amd.gpu_csr_add_f32(A, B)` for the default workload (C2:
two 2^20 x 2^20 CSR matrices with rescaled Zipf(1.6) row lengths, 16.7M nonzeros each).
A call includes result allocation from the device pool, the kernels and the readback of
the result length; it returns once the length is known, while its last kernel (the write
pass) still runs on the stream, so one call's write pass overlaps the next call's host
work.  The timed region ends with a device synchronize, so every step's kernels are inside
it.  Steps rotate over several independent copies of the operands so that no step re-reads
inputs still resident in the 256 MB Infinity Cache.

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

Workload c4 (ESC SpGEMM, C = A*A on the R-MAT 2^20 operand) reports GFLOP/s = 2*P / call
time, P = number of intermediate products; its roofline bytes are
4*(n+1) + 8*nnzA + 8*P (B's gathered entries) + 8*(n+1) + 8*nnzC, and its CPU baseline is
the row-parallel C SpGEMM of oracle/ on a random row sample.

Workloads mtx and tns run the same measurements on local files, paired as the reference's
sweeps pair them (benchmarks/csr_add.py:45-124, benchmarks/frostt_tensors_add.py:52-149):
consecutive .mtx files clipped to a common shape, through csr_add and csr_mul; each .tns
file with its copy shifted by one along every mode, through csf_add and coo3d_add.

Workloads c5 (csf_add), c5coo (coo3d_add), c2coo (coo_add), c3coo (coo_mul), c2dcsr
(dcsr_add) and c3dcsr (dcsr_mul) report GB/s of algorithmic bytes: CSF3 and DCSR count
every level array of A, B and C once; COO3 16 bytes and COO 12 bytes per entry of A, B and
C.  c5inner / c5innercoo (inner_prod / inner_prod_coo of the C5 operands) count every array
of A and B once plus the 4-byte result; c2coocsr (coo_csr_add of the C2 operands, B as COO)
counts A and C as CSR and B as COO.
"""

from __future__ import annotations

import argparse
import ctypes
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
    "c2": dict(op="add", kernel="csr_partition_kernel (with the row pass) + "
                              "csr_pair_count_kernel (pair search) + csr_write_kernel<Union> "
                              "(one call's device pipeline)",
               desc="C2 csr_add f32 2^20x2^20, Zipf(1.6) rows rescaled to mean 16 "
                    "(16.7M nnz each), seeds 1/2"),
    "c3": dict(op="mul", kernel="csr_partition_kernel + csr_write_kernel<Intersect> (spread) "
                              "+ csr_compact_kernel (one call's device pipeline)",
               desc="C3 csr_mul f32 2^20x2^20, A as C2, B = 50% of A + fresh columns "
                    "(seed 3)"),
    "c5": dict(op="csf_add", kernel="three chained level merges (csr_partition_kernel + "
                                   "csr_pair_count_kernel + csr_write_kernel per level)",
               desc="C5 csf_add f32, two CSF3 tensors of shape (200000, 100000, 1000), 20M "
                    "draws each (mode 0 Zipf(1.3), modes 1-2 uniform), deduplicated, seeds 1/2"),
    "c5coo": dict(op="coo3d_add", kernel="coo3_keys_kernel (row offsets, (j, k) keys) + "
                                         "csr_partition_kernel + csr_pair_count_kernel + "
                                         "csr_write_kernel<Union> (rows out, keys split)",
                  desc="C5 as COO3: coo3d_add f32 of the same (i, j, k) tuples"),
    "c3coo": dict(op="coo_mul", kernel="coo_row_offsets_kernel + csr_partition_kernel + "
                                      "csr_write_kernel<Intersect> (spread, rows out) + "
                                      "csr_compact_kernel",
                  desc="C3 as COO: coo_mul f32 of the C3 operands' (i, j) tuples"),
    "c2coo": dict(op="coo_add", kernel="coo_row_offsets_kernel + csr_partition_kernel + "
                                      "csr_pair_count_kernel + csr_write_kernel<Union> (rows out)",
                  desc="C2 as COO: coo_add f32 of the C2 operands' (i, j) tuples"),
    "c2add3": dict(op="add3", kernel="fused three-way merge (csr3_partition_kernel + "
                                    "csr3_count_kernel + csr3_write_kernel)",
                   desc="csr_add_3 f32: three C2 operands (Zipf(1.6) rows, 16.7M nnz each, "
                        "seeds 1, 2, 4)"),
    "c2dcsr": dict(op="dcsr_add", kernel="two chained level merges (csr_partition_kernel + "
                                        "csr_pair_count_kernel + csr_write_kernel per level)",
                   desc="C2 as DCSR: dcsr_add f32 of the C2 operands with empty rows "
                        "dropped"),
    "c5inner": dict(op="inner_prod", kernel="csf_row_offsets_kernel + csf_keys_kernel + "
                                          "csr_partition_kernel + csr_write_kernel<Intersect> "
                                          "(spread) + dot_tiles_kernel + dot_final_kernel",
                    desc="inner_prod f32 of the C5 CSF3 operands: sum of a*b over the "
                         "(i, j, k) both hold"),
    "c5innercoo": dict(op="inner_prod_coo", kernel="coo3_keys_kernel + csr_partition_kernel + "
                                                   "csr_write_kernel<Intersect> (spread) + "
                                                   "dot_tiles_kernel + dot_final_kernel",
                       desc="inner_prod_coo f32 of the C5 operands as COO3"),
    "c2coocsr": dict(op="coo_csr_add", kernel="coo_row_offsets_kernel + csr_partition_kernel "
                                             "(with the row pass) + csr_pair_count_kernel + "
                                             "csr_write_kernel<Union>",
                     desc="coo_csr_add f32: the C2 operands, A as CSR and B as COO"),
    "c3dcsr": dict(op="dcsr_mul", kernel="two chained level merges + row compaction",
                   desc="C3 as DCSR: dcsr_mul f32 of the C3 operands with empty rows "
                        "dropped"),
    "c4sssmm": dict(op="sssmm", kernel="hash tables + probe_kernel + output (one call's "
                                       "device pipeline, host readback gaps excluded)",
                    desc="sssmm f32: A * A masked by A on the C4 operand (R-MAT 2^20); "
                         "GFLOP/s = 3 FLOP (two multiplies, one add) per term"),
    "c4": dict(op="spgemm", kernel="long_hist_kernel + long_runs_kernel (run descriptors) + "
                                 "dense/bitmap/sort unit kernels + copy_units_kernel (staged output) and the "
                                 "sizing kernels "
                                 "(one call's device pipeline, host readback gaps excluded)",
               desc="C4 ESC SpGEMM C=A*A f32, R-MAT 2^20 (a,b,c,d)=(.57,.19,.19,.05), "
                    "8*2^20 draws deduplicated, no vertex permutation, values U[0.5,1.5], "
                    "seed 1; int64 result offsets"),
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model():
    """The host CPU's model name (first `model name` of /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def host_cores():
    return max(1, min(len(os.sched_getaffinity(0)), 64))


def compact(workload, line):
    """The fields of one workload's line that go into the default run's `workloads` list."""
    rec = {
        "workload": workload,
        "config": line["config"]["workload"],
        "metric": "GFLOP/s" if line["unit"] == "GFLOP/s" else "effective HBM GB/s",
        "value": line["value"],
        "unit": line["unit"],
        "ms_per_call": line["ms_per_step"],
        "steps": line["steps"],
        "roofline": line["roofline"],
        "cpu_baseline": line["cpu_baseline"],
    }
    if line["unit"] == "GB/s":
        rec["percent_of_peak_hbm"] = round(100.0 * line["value"] / PEAK_HBM_GBS, 2)
    cpu = line["cpu_baseline"]
    if cpu:
        rec["gpu_over_cpu"] = round(line["value"] / cpu["value"], 1)
    for key in ("products", "flops_per_step", "nnz_c", "algorithmic_bytes_per_step"):
        if key in line["config"]:
            rec[key] = line["config"][key]
    return rec


def collect_garbage():
    """A full collection of Python's garbage, run before the warmup steps rather than right
    before the timed region: it keeps the device idle for tens of milliseconds, and calls
    timed right after such a pause ran slower (C2: 170.0 instead of 159.2 us per call over
    50 steps), as if the device were still waking up."""
    import gc

    gc.collect()


def timed_steps(step, steps):
    """Wall seconds of `steps` calls step(0) .. step(steps - 1), synchronized with the device
    on both sides.  Python's garbage collector (run before the warmup, collect_garbage) is
    paused inside (as timeit does), so a collection cannot land in the timed region; results
    are still released as soon as they are dropped (reference counting)."""
    import gc

    import torch

    torch.cuda.synchronize()
    enabled = gc.isenabled()
    gc.disable()
    try:
        start = time.perf_counter()
        for i in range(steps):
            step(i)
        torch.cuda.synchronize()
        return time.perf_counter() - start
    finally:
        if enabled:
            gc.enable()


def make_operands(workload):
    from nacho_amd import synth

    if workload == "c2":
        return synth.c2_operands()
    if workload == "c2add3":
        return tuple(synth.zipf_csr(synth.C2_ROWS, s) for s in (1, 2, 4))
    return synth.c3_operands()


def traffic_from_profiles(workload, family="csr_merge"):
    """(measured HBM bytes per call of the device pipeline, the commit the counters were
    taken on) from profiles/, or (None, None) when that workload was not profiled."""
    path = REPO / "profiles" / f"{family}_{workload}_traffic.json"
    if workload is None or not path.exists():
        return None, None
    try:
        rec = json.loads(path.read_text())
    except (OSError, ValueError):
        return None, None
    return rec.get("hbm_bytes_per_launch"), rec.get("commit")


_COPY_CEILING = {}


def copy_ceiling(device):
    """Device-copy rates on this GPU, measured once per run: the library's streaming copy
    kernel (nacho_device_copy) and torch's copy_, each moving 1 GiB in and 1 GiB out,
    10 timed copies after 3 warm-up ones, HIP events on the stream the copies run on."""
    if _COPY_CEILING:
        return _COPY_CEILING
    import torch

    from nacho_amd import _lib

    lib = _lib.load()
    n = 1 << 28  # 1 GiB of float32
    src = torch.ones(n, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream(device)

    def rate(copy):
        for _ in range(3):
            copy()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(10):
            copy()
        stop.record(stream)
        stop.synchronize()
        return 10 * 2 * 4 * n / (start.elapsed_time(stop) * 1e-3) / 1e9

    def kernel_copy():
        rc = lib.nacho_device_copy(ctypes.c_void_p(dst.data_ptr()),
                                   ctypes.c_void_p(src.data_ptr()), 4 * n,
                                   ctypes.c_void_p(stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(_lib.error_string(rc))

    _COPY_CEILING["kernel_gbs"] = round(rate(kernel_copy), 1)
    _COPY_CEILING["torch_copy_gbs"] = round(rate(lambda: dst.copy_(src)), 1)
    del src, dst
    torch.cuda.empty_cache()
    log(f"copy ceiling: nacho_device_copy {_COPY_CEILING['kernel_gbs']} GB/s, torch copy_ "
        f"{_COPY_CEILING['torch_copy_gbs']} GB/s (1 GiB read + 1 GiB written)")
    return _COPY_CEILING


def roofline(device, kernel, achieved, kernel_avg_ms, traffic_key, family):
    """The line's roofline object: HBM-bound, against the MI355X peak, with the measured
    copy ceilings and the counter-measured traffic (and its commit) of the workload."""
    traffic, commit = traffic_from_profiles(traffic_key, family)
    ceiling = copy_ceiling(device)
    return {
        "bound": "hbm",
        "kernel": kernel,
        "achieved": round(achieved, 2),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_HBM_GBS, 4),
        "traffic": traffic,
        "traffic_commit": commit,
        "kernel_avg_us": round(kernel_avg_ms * 1e3, 2),
        "copy_ceiling_gbs": ceiling["kernel_gbs"],
        "torch_copy_gbs": ceiling["torch_copy_gbs"],
        "frac_of_copy_ceiling": round(achieved / ceiling["kernel_gbs"], 4),
    }


def cpu_baseline(workload, op, operands, rows, bytes_per_call, budget_s):
    """Time the oracle's C restatement of the reference CPU kernel on this host."""
    from oracle import oracle

    cores = host_cores()
    times = []
    start = time.perf_counter()
    while time.perf_counter() - start < budget_s and len(times) < 50:
        t = {}
        if op == "add3":
            oracle.port_csr_add3(rows, *operands, timing=t, nthreads=cores)
        else:
            oracle.port_csr_binary(op, rows, *operands[0], *operands[1], nthreads=cores,
                                   timing=t)
        times.append(t["seconds"])
    times.sort()
    trimmed = times[1:-1] if len(times) > 4 else times
    sec = sum(trimmed) / len(trimmed)
    return {
        "value": round(bytes_per_call / sec / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"{len(times)} full {workload} calls of the C restatement "
                  f"(oracle/nacho_oracle.c, one partition per thread), mean of the middle "
                  f"{len(trimmed)}: {sec * 1e3:.1f} ms/call",
    }


def spgemm_products(pos, crd):
    """P = sum over A entries (i, j) of |row j| (A times A)."""
    import numpy as np

    lens = np.diff(pos.astype(np.int64))
    return int(lens[crd].sum())


def spgemm_cpu_baseline(pos, crd, val, budget_s):
    """Row-parallel CPU SpGEMM with the reference's ESC result semantics (oracle/), on a
    uniform random sample of A's rows sized to take about `budget_s` in total."""
    import numpy as np

    from oracle import oracle

    n = len(pos) - 1
    cores = host_cores()
    lens = np.diff(pos.astype(np.int64))
    rng = np.random.default_rng(99)

    def run(frac):
        rows = np.sort(rng.choice(n, size=max(1, int(n * frac)), replace=False))
        sl = lens[rows]
        sp = np.zeros(len(rows) + 1, np.int64)
        sp[1:] = np.cumsum(sl)
        idx = np.repeat(pos[rows].astype(np.int64) - sp[:-1], sl) + np.arange(sp[-1])
        sub = (sp.astype(np.int32), crd[idx], val[idx])
        prods = int(lens[sub[1]].sum())
        t0 = time.perf_counter()
        oracle.port_spgemm(len(rows), n, n, *sub, pos, crd, val, nthreads=cores)
        return prods, time.perf_counter() - t0, len(rows)

    p0, t0, _ = run(1 / 512)
    rate = p0 / max(t0, 1e-6)
    total_p = lens[crd].sum()
    frac = min(1.0, max(1 / 512, rate * budget_s / 2 / total_p))
    samples = [run(frac) for _ in range(2)]
    prods = sum(x[0] for x in samples)
    sec = sum(x[1] for x in samples)
    return {
        "value": round(2 * prods / sec / 1e9, 3),
        "unit": "GFLOP/s",
        "cores": cores,
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"2 runs of A[rows] @ A on uniform random samples of {samples[0][2]} rows "
                  f"({frac:.4f} of rows; {prods} products in {sec:.1f} s) with the "
                  f"row-parallel C SpGEMM (oracle/nacho_oracle.c, float64 sums)",
    }


def bench_spgemm(args, device):
    import torch

    import nacho_amd
    from nacho_amd import synth

    spec = WORKLOADS["c4"]
    t0 = time.perf_counter()
    pos, crd, val = synth.c4_operand()
    n = len(pos) - 1
    P = spgemm_products(pos, crd)
    log(f"generated c4: n={n} nnzA={len(crd)} products={P} in {time.perf_counter() - t0:.1f}s")

    def upload():
        t = (torch.from_numpy(x).to(device) for x in (pos, crd, val))
        return nacho_amd.CSR_gpu(*t, torch.tensor([n, n], dtype=torch.int32))

    copies = [upload() for _ in range(2)]
    fn = nacho_amd.gpu_spgemm64_f32
    z = fn(copies[0], copies[0])
    torch.cuda.synchronize()
    nnz_c = int(z.dim_j_indices.numel())
    del z
    flops = 2 * P
    # algorithmic bytes: A as left operand, B's gathered entries, the int64-offset result
    compulsory = 4 * (n + 1) + 8 * len(crd) + 8 * (n + 1) + 8 * nnz_c
    alg_bytes = compulsory + 8 * P
    log(f"nnzC={nnz_c} flops/call={flops} algorithmic bytes/call={alg_bytes}")

    collect_garbage()
    nacho_amd.set_kernel_timing(True)
    for i in range(args.warmup):
        fn(copies[i % 2], copies[i % 2])
    torch.cuda.synchronize()
    kernel_ms = []
    for i in range(args.steps):
        fn(copies[i % 2], copies[i % 2])
        kernel_ms.append(nacho_amd.last_kernel_ms())
    nacho_amd.set_kernel_timing(False)
    torch.cuda.synchronize()

    elapsed = timed_steps(lambda i: fn(copies[i % 2], copies[i % 2]), args.steps)
    ms_per_step = elapsed * 1e3 / args.steps
    value = flops / (ms_per_step * 1e-3) / 1e9
    kernel_avg_ms = sum(kernel_ms) / len(kernel_ms)
    achieved = alg_bytes / (kernel_avg_ms * 1e-3) / 1e9
    log(f"pipeline avg {kernel_avg_ms:.2f} ms -> {achieved:.0f} GB/s; call {ms_per_step:.2f} ms "
        f"-> {value:.1f} GFLOP/s")

    cpu = None
    if args.cpu_budget > 0:
        cpu = spgemm_cpu_baseline(pos, crd, val, args.cpu_budget)
        log(f"cpu baseline {cpu['value']} GFLOP/s on {cpu['cores']} threads")
    nacho_amd.release_cached_memory()

    return {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded generators in nacho_amd/synth.py)",
        "config": {
            "workload": spec["desc"],
            "rows": n,
            "nnz_a": len(crd),
            "products": P,
            "nnz_c": nnz_c,
            "flops_per_step": flops,
            "algorithmic_bytes_per_step": alg_bytes,
            "compulsory_bytes_per_step": compulsory,
            "parallelism": "single GPU",
        },
        "roofline": roofline(device, spec["kernel"], achieved, kernel_avg_ms, "c4",
                             "spgemm"),
        "cpu_baseline": cpu,
        "gpu_over_cpu": round(value / cpu["value"], 1) if cpu else None,
    }


def sssmm_cpu_baseline(pos, crd, budget_s):
    """The oracle's row-parallel masked SpGEMM (A, A, A) on a uniform random row sample sized
    to take about `budget_s`; unit values, so the result values count the terms."""
    import numpy as np

    from oracle import oracle

    n = len(pos) - 1
    cores = host_cores()
    ones = np.ones(len(crd), np.float32)
    rng = np.random.default_rng(98)
    a = (pos, crd, ones)

    def run(frac):
        rows = np.sort(rng.choice(n, size=max(1, int(n * frac)), replace=False)).astype(np.int32)
        t0 = time.perf_counter()
        _, _, v = oracle.port_sssmm(n, n, a, a, a, row_list=rows, nthreads=cores)
        return float(np.sum(v, dtype=np.float64)), time.perf_counter() - t0, len(rows)

    _, s_small, _ = run(1 / 512)
    frac = min(1.0, max(1 / 512, (budget_s / 2) / max(s_small, 1e-6) / 512))
    samples = [run(frac) for _ in range(2)]
    terms = sum(x[0] for x in samples)
    sec = sum(x[1] for x in samples)
    return {
        "value": round(3 * terms / sec / 1e9, 3),
        "unit": "GFLOP/s",
        "cores": cores,
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"2 runs of the row-parallel C masked SpGEMM (oracle/nacho_oracle.c, dense "
                  f"mask marker, float64 sums) on uniform random samples of {samples[0][2]} "
                  f"rows ({frac:.4f} of rows; {int(terms)} terms in {sec:.1f} s)",
    }


def bench_sssmm(args, device):
    """c4sssmm: the masked product A * A masked by A on the C4 operand (the reference's
    sssmm benchmark runs A, A, A for square matrices, benchmarks/sssmm.py:13-15)."""
    import numpy as np
    import torch

    import nacho_amd
    from nacho_amd import synth

    spec = WORKLOADS["c4sssmm"]
    t0 = time.perf_counter()
    pos, crd, val = synth.c4_operand()
    n = len(pos) - 1
    lens = np.diff(pos.astype(np.int64))
    colcnt = np.bincount(crd, minlength=n).astype(np.int64)
    rows = np.repeat(np.arange(n), lens)
    la, lb = lens[rows], colcnt[crd]
    probes = int(np.where((la > 0) & (lb > 0), np.minimum(la, lb), 0).sum())
    log(f"generated c4sssmm: n={n} nnz={len(crd)} probes={probes} "
        f"in {time.perf_counter() - t0:.1f}s")

    def upload(values):
        t = (torch.from_numpy(x).to(device) for x in (pos, crd, values))
        return nacho_amd.CSR_gpu(*t, torch.tensor([n, n], dtype=torch.int32))

    ones = upload(np.ones(len(crd), np.float32))
    zc = nacho_amd.gpu_sssmm_f32(ones, ones, ones)
    terms = int(zc.values.double().sum().item())  # unit values: each entry counts its terms
    del zc, ones
    copies = [upload(val) for _ in range(2)]
    fn = nacho_amd.gpu_sssmm_f32
    z = fn(copies[0], copies[0], copies[0])
    torch.cuda.synchronize()
    nnz_z = int(z.dim_j_indices.numel())
    del z
    flops = 3 * terms
    operand = 4 * (n + 1) + 8 * len(crd)
    alg_bytes = 3 * operand + 4 * (n + 1) + 8 * nnz_z + 8 * probes
    log(f"nnzZ={nnz_z} terms={terms} flops/call={flops} algorithmic bytes/call={alg_bytes}")

    collect_garbage()
    nacho_amd.set_kernel_timing(True)
    for i in range(args.warmup):
        fn(*(copies[i % 2],) * 3)
    torch.cuda.synchronize()
    kernel_ms = []
    for i in range(args.steps):
        fn(*(copies[i % 2],) * 3)
        kernel_ms.append(nacho_amd.last_kernel_ms())
    nacho_amd.set_kernel_timing(False)
    torch.cuda.synchronize()
    ms_per_step = timed_steps(lambda i: fn(*(copies[i % 2],) * 3), args.steps) * 1e3 / args.steps
    value = flops / (ms_per_step * 1e-3) / 1e9
    kernel_avg_ms = sum(kernel_ms) / len(kernel_ms)
    achieved = alg_bytes / (kernel_avg_ms * 1e-3) / 1e9
    log(f"pipeline avg {kernel_avg_ms:.3f} ms -> {achieved:.0f} GB/s; call {ms_per_step:.3f} ms "
        f"-> {value:.1f} GFLOP/s")

    cpu = None
    if args.cpu_budget > 0:
        cpu = sssmm_cpu_baseline(pos, crd, args.cpu_budget)
        log(f"cpu baseline {cpu['value']} GFLOP/s on {cpu['cores']} threads")
    nacho_amd.release_cached_memory()
    return {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded generators in nacho_amd/synth.py)",
        "config": {
            "workload": spec["desc"],
            "rows": n,
            "nnz_a": len(crd),
            "probes": probes,
            "terms": terms,
            "nnz_z": nnz_z,
            "flops_per_step": flops,
            "algorithmic_bytes_per_step": alg_bytes,
            "parallelism": "single GPU",
        },
        "roofline": roofline(device, spec["kernel"], achieved, kernel_avg_ms, "c4sssmm",
                             "sssmm"),
        "cpu_baseline": cpu,
        "gpu_over_cpu": round(value / cpu["value"], 1) if cpu else None,
    }


def csf_bytes(levels_list):
    """Every array of every CSF3 tensor once: crd_i, pos_j, crd_j, pos_k, crd_k, val."""
    total = 0
    for levels in levels_list:
        ci, pj, cj, pk, ck = levels
        total += 4 * (len(ci) + len(pj) + len(cj) + len(pk) + 2 * len(ck))
    return total


def dcsr_levels(pos, crd):
    """DCSR levels (crd_i, pos_j, crd_j) of a CSR matrix: empty rows dropped."""
    import numpy as np

    lengths = np.diff(np.asarray(pos, np.int64))
    present = np.flatnonzero(lengths > 0)
    pj = np.zeros(len(present) + 1, np.int64)
    pj[1:] = np.cumsum(lengths[present])
    return present.astype(np.int32), pj.astype(np.int32), np.asarray(crd, np.int32)


def bench_tuple_workload(args, device, workload, prepared=None):
    """c5 (csf_add), c5coo (coo3d_add), c2coo (coo_add), c2dcsr / c3dcsr (dcsr_add /
    dcsr_mul): element-wise merges of coordinate trees or tuples; one step = one call with
    operands resident in HBM.  `prepared` = (spec, operands, shape, data) measures csf_add
    (workload c5) or coo3d_add (c5coo) on given (i, j, k) operands (the file workloads)."""
    import numpy as np
    import torch

    import nacho_amd
    from nacho_amd import synth
    from nacho_amd.convert import csf3_levels

    spec = WORKLOADS[workload]
    data = "synthetic (seeded generators in nacho_amd/synth.py)"
    traffic_key = workload
    t0 = time.perf_counter()
    if prepared is not None:
        spec, ops_np, shape, data = prepared
        traffic_key = None
    elif workload in ("c2dcsr", "c3dcsr"):
        ops = synth.c2_operands() if workload == "c2dcsr" else synth.c3_operands()
        ops_np = [(dcsr_levels(p, c), v) for p, c, v in ops]
        shape = (len(ops[0][0]) - 1, len(ops[0][0]) - 1)
    elif workload in ("c2coo", "c3coo", "c2coocsr"):
        ops = synth.c3_operands() if workload == "c3coo" else synth.c2_operands()
        (pa, ca, va), (pb, cb, vb) = ops
        rows = len(pa) - 1
        ia = np.repeat(np.arange(rows, dtype=np.int32), np.diff(pa))
        ib = np.repeat(np.arange(rows, dtype=np.int32), np.diff(pb))
        ops_np = [((ia, ca), va), ((ib, cb), vb)]
        shape = (rows, rows)
        if workload == "c2coocsr":  # A keeps its row offsets
            ops_np[0] = ((pa, ca), va)
    else:
        (ac, av), (bc, bv) = synth.c5_operands()
        ops_np = [(tuple(ac[:, d] for d in range(3)), av), (tuple(bc[:, d] for d in range(3)), bv)]
        shape = synth.C5_SHAPE
    if prepared is None:
        log(f"generated {workload}: nnzA={len(ops_np[0][1])} nnzB={len(ops_np[1][1])} "
            f"in {time.perf_counter() - t0:.1f}s")

    def upload(crd, val, k):
        t = [torch.from_numpy(np.ascontiguousarray(c, dtype=np.int32)).to(device) for c in crd]
        v = torch.from_numpy(np.ascontiguousarray(val, dtype=np.float32)).to(device)
        dims = torch.tensor(list(shape), dtype=torch.int32)
        if workload in ("c2dcsr", "c3dcsr"):
            return nacho_amd.DCSR_gpu(t[0], t[1], t[2], v, dims)
        if workload in ("c2coo", "c3coo", "c2coocsr"):
            if workload == "c2coocsr" and k == 0:  # A: CSR (row offsets, columns)
                return nacho_amd.CSR_gpu(t[0], t[1], v, dims)
            return nacho_amd.COO_gpu(t[0], t[1], v, dims)
        if workload in ("c5coo", "c5innercoo"):
            return nacho_amd.COO3_gpu(t[0], t[1], t[2], v, dims)
        levels = csf3_levels(np.stack(crd, axis=1))
        lv = [torch.from_numpy(np.ascontiguousarray(x, dtype=np.int32)).to(device) for x in levels]
        return nacho_amd.CSF3_gpu(*lv, v, dims)

    copies = [tuple(upload(*o, k) for k, o in enumerate(ops_np)) for _ in range(ROTATE)]
    fn = {"c2coo": nacho_amd.gpu_coo_add_f32, "c3coo": nacho_amd.gpu_coo_mul_f32,
          "c5coo": nacho_amd.gpu_coo3d_add_f32,
          "c5": nacho_amd.gpu_csf_add_f32, "c2dcsr": nacho_amd.gpu_dcsr_add_f32,
          "c3dcsr": nacho_amd.gpu_dcsr_mul_f32, "c5inner": nacho_amd.gpu_inner_prod_f32,
          "c5innercoo": nacho_amd.gpu_inner_prod_coo_f32,
          "c2coocsr": nacho_amd.gpu_coo_csr_add_f32}[workload]
    z = fn(*copies[0])
    torch.cuda.synchronize()
    nnz = [len(ops_np[0][1]), len(ops_np[1][1]), int(z.values.numel())]
    if workload == "c5":
        lz = [z.dim_i_indices.numel(), z.dim_j_offsets.numel(), z.dim_j_indices.numel(),
              z.dim_k_offsets.numel(), z.dim_k_indices.numel()]
        alg_bytes = csf_bytes([csf3_levels(np.stack(o[0], axis=1)) for o in ops_np])
        alg_bytes += 4 * (sum(lz) + lz[4])
    elif workload == "c5inner":
        # every array of A and B once, and the one result value
        alg_bytes = csf_bytes([csf3_levels(np.stack(o[0], axis=1)) for o in ops_np]) + 4
    elif workload == "c5innercoo":
        alg_bytes = 16 * (nnz[0] + nnz[1]) + 4
    elif workload == "c2coocsr":
        # A: pos, crd, val; B: i, j, val; C: pos, crd, val
        rows = shape[0]
        alg_bytes = 8 * (rows + 1) + 8 * nnz[0] + 12 * nnz[1] + 8 * nnz[2]
    elif workload in ("c2dcsr", "c3dcsr"):
        # crd_i, pos_j, crd_j and values of A, B and C
        alg_bytes = sum(4 * (len(o[0][0]) + len(o[0][1]) + 2 * len(o[0][2])) for o in ops_np)
        alg_bytes += 4 * (z.dim_i_indices.numel() + z.dim_j_offsets.numel()
                          + 2 * z.dim_j_indices.numel())
    else:
        alg_bytes = (12 if workload in ("c2coo", "c3coo") else 16) * sum(nnz)
    del z
    log(f"nnzC={nnz[2]} algorithmic bytes/call={alg_bytes}")

    collect_garbage()
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
    ms_per_step = timed_steps(lambda i: fn(*copies[i % ROTATE]), args.steps) * 1e3 / args.steps
    value = alg_bytes / (ms_per_step * 1e-3) / 1e9
    kernel_avg_ms = sum(kernel_ms) / len(kernel_ms)
    achieved = alg_bytes / (kernel_avg_ms * 1e-3) / 1e9
    log(f"kernel avg {kernel_avg_ms * 1e3:.1f} us -> {achieved:.0f} GB/s; "
        f"call {ms_per_step * 1e3:.1f} us -> {value:.0f} GB/s")

    cpu = None
    if args.cpu_budget > 0:
        from oracle import oracle

        cores = host_cores()
        times = []
        if workload in ("c5", "c5inner"):
            levels = [csf3_levels(np.stack(o[0], axis=1)) for o in ops_np]
        begin = time.perf_counter()
        while time.perf_counter() - begin < args.cpu_budget and len(times) < 20:
            t = {}
            if workload in ("c2dcsr", "c3dcsr"):
                oracle.port_dcsr_binary("add" if workload == "c2dcsr" else "mul",
                                        ops_np[0][0], ops_np[0][1], ops_np[1][0],
                                        ops_np[1][1], timing=t, nthreads=cores)
            elif workload == "c5":
                oracle.port_csf3_union(levels[0], ops_np[0][1], levels[1], ops_np[1][1],
                                       timing=t, nthreads=cores)
            elif workload == "c5inner":
                oracle.port_csf3_inner(levels[0], ops_np[0][1], levels[1], ops_np[1][1],
                                       timing=t, nthreads=cores)
            elif workload == "c5innercoo":
                oracle.port_coo3_inner(ops_np[0][0], ops_np[0][1], ops_np[1][0], ops_np[1][1],
                                       timing=t, nthreads=cores)
            elif workload == "c2coocsr":
                # the C restatement of csr_add on the same operands (B's row offsets given)
                pb = np.zeros(shape[0] + 1, np.int64)
                np.add.at(pb, np.asarray(ops_np[1][0][0], np.int64) + 1, 1)
                pb = np.cumsum(pb).astype(np.int32)
                oracle.port_csr_binary("add", shape[0], ops_np[0][0][0], ops_np[0][0][1],
                                       ops_np[0][1], pb, ops_np[1][0][1], ops_np[1][1],
                                       nthreads=cores, timing=t)
            else:
                oracle.port_coo_binary("mul" if workload == "c3coo" else "add", ops_np[0][0],
                                       ops_np[0][1], ops_np[1][0], ops_np[1][1],
                                       nthreads=cores, timing=t)
            times.append(t["seconds"])
        sec = sorted(times)[len(times) // 2]
        cpu = {
            "value": round(alg_bytes / sec / 1e9, 3),
            "unit": "GB/s",
            "cores": cores,
            "cpu_model": cpu_model(),
            "kind": "port",
            "sample": f"{len(times)} full {workload} calls of the C restatement "
                      f"(oracle/nacho_oracle.c, one partition per thread), "
                      f"median {sec * 1e3:.1f} ms/call",
        }
        log(f"cpu baseline {cpu['value']} GB/s on {cpu['cores']} threads")

    return {
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
        "data": data,
        "config": {
            "workload": spec["desc"],
            "nnz_a": nnz[0],
            "nnz_b": nnz[1],
            "nnz_c": nnz[2],
            "algorithmic_bytes_per_step": alg_bytes,
            "percent_of_peak_hbm": round(100.0 * value / PEAK_HBM_GBS, 2),
            "parallelism": "single GPU",
        },
        "roofline": roofline(device, spec["kernel"], achieved, kernel_avg_ms, traffic_key,
                             "tuple_merge"),
        "cpu_baseline": cpu,
    }


def bench_csr(args, device, workload, prepared=None):
    """c2 (csr_add), c3 (csr_mul), c2add3 (csr_add_3): one step = one call with operands
    resident in HBM, rotating over ROTATE copies.  `prepared` = (spec, operands, (rows,
    cols), data) runs the same measurement on given operands (the file workloads)."""
    import numpy as np
    import torch

    import nacho_amd
    from nacho_amd import synth

    t0 = time.perf_counter()
    if prepared is None:
        spec = WORKLOADS[workload]
        operands_np = make_operands(workload)
        rows = cols = len(operands_np[0][0]) - 1
        data = "synthetic (seeded generators in nacho_amd/synth.py)"
        log(f"generated {workload}: rows={rows} "
            f"nnz={[len(o[1]) for o in operands_np]} in {time.perf_counter() - t0:.1f}s")
    else:
        spec, operands_np, (rows, cols), data = prepared
    a_np, b_np = operands_np[0], operands_np[1]

    def upload(t):
        pos, crd, val = (torch.from_numpy(np.ascontiguousarray(x)).to(device) for x in t)
        return nacho_amd.CSR_gpu(pos, crd, val, torch.tensor([rows, cols], dtype=torch.int32))

    copies = [tuple(upload(o) for o in operands_np) for _ in range(ROTATE)]
    fn = {"add": nacho_amd.gpu_csr_add_f32, "mul": nacho_amd.gpu_csr_mul_f32,
          "add3": nacho_amd.gpu_csr_add_3_f32}[spec["op"]]

    z = fn(*copies[0])
    torch.cuda.synchronize()
    nnz_c = int(z.dim_j_indices.numel())
    del z
    alg_bytes = synth.csr_bytes(rows, len(a_np[1]), len(b_np[1]), nnz_c)
    if spec["op"] == "add3":  # the third operand's offsets and entries
        alg_bytes += 4 * (rows + 1) + 8 * len(operands_np[2][1])
    log(f"nnzC={nnz_c} algorithmic bytes/call={alg_bytes}")

    # warmup, then per-launch kernel durations (HIP events on the launch stream)
    collect_garbage()
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
    elapsed = timed_steps(lambda i: fn(*copies[i % ROTATE]), args.steps)
    ms_per_step = elapsed * 1e3 / args.steps
    value = alg_bytes / (ms_per_step * 1e-3) / 1e9

    kernel_avg_ms = sum(kernel_ms) / len(kernel_ms)
    achieved = alg_bytes / (kernel_avg_ms * 1e-3) / 1e9
    log(f"kernel avg {kernel_avg_ms * 1e3:.1f} us -> {achieved:.0f} GB/s; "
        f"call {ms_per_step * 1e3:.1f} us -> {value:.0f} GB/s")

    cpu = None
    if args.cpu_budget > 0:
        cpu = cpu_baseline(workload, spec["op"], operands_np, rows, alg_bytes,
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
        "data": data,
        "config": {
            "workload": spec["desc"],
            "rows": rows,
            "cols": cols,
            "nnz_operands": [len(o[1]) for o in operands_np],
            "nnz_a": len(a_np[1]),
            "nnz_b": len(b_np[1]),
            "nnz_c": nnz_c,
            "algorithmic_bytes_per_step": alg_bytes,
            "percent_of_peak_hbm": round(100.0 * value / PEAK_HBM_GBS, 2),
            "parallelism": "single GPU",
        },
        "roofline": roofline(device, spec["kernel"], achieved, kernel_avg_ms, workload,
                             "csr_merge"),
        "cpu_baseline": cpu,
    }
    return line


def bench_files(args, device):
    """The real-data workloads on local files (one line; the first measurement is its
    value, the others are listed under `workloads`).

    mtx: consecutive pairs of the given Matrix Market files (a single file is paired with
    itself), each clipped to a common shape as the reference's matrix sweep does
    (benchmarks/csr_add.py:57-65), then csr_add, csr_mul and coo_csr_add (the second
    matrix as COO).
    tns: each FROSTT file as A (sorted, repeats summed) and its shifted copy as B
    (benchmarks/frostt_tensors_add.py:62-64), then csf_add (CSF3), coo3d_add (COO3),
    inner_prod (CSF3) and inner_prod_coo (COO3)."""
    import numpy as np

    from nacho_amd import io

    paths = [Path(p) for p in args.files]
    if not paths:
        raise SystemExit(f"--workload {args.workload} needs --files")
    for p in paths:
        if not p.is_file():
            raise SystemExit(f"no such file: {p}")
    lines = []
    if args.workload == "mtx":
        mats = []
        for p in paths:
            t0 = time.perf_counter()
            mats.append(io.parse_matrix(p, device="cpu"))
            log(f"parsed {p.name}: {tuple(mats[-1].shape)} nnz={mats[-1].values().numel()} "
                f"in {time.perf_counter() - t0:.1f}s")
        pairs = list(zip(range(len(paths) - 1), range(1, len(paths)))) or [(0, 0)]
        for i, j in pairs:
            rows, cols, a, b = io.clip_to_common_shape(mats[i], mats[j])
            names = f"{paths[i].name} and {paths[j].name}"
            for op, kernel in (("add", "csr_add"), ("mul", "csr_mul")):
                spec = dict(WORKLOADS["c2" if op == "add" else "c3"])
                spec["op"] = op
                spec["desc"] = (f"{kernel} f32 of {names} clipped to {rows}x{cols} "
                                f"(nnz {len(a[1])} + {len(b[1])})")
                data = f"local Matrix Market files: {names}"
                lines.append(bench_csr(args, device, "mtx",
                                       prepared=(spec, (a, b), (rows, cols), data)))
            # the same pair with the right operand as COO (benchmarks/coo_csr_add.py:25-44)
            spec = dict(WORKLOADS["c2coocsr"])
            spec["desc"] = (f"coo_csr_add f32 of {names} clipped to {rows}x{cols}, the "
                            f"second as COO (nnz {len(a[1])} + {len(b[1])})")
            bi = np.repeat(np.arange(rows, dtype=np.int32), np.diff(np.asarray(b[0])))
            ops = [((a[0], a[1]), a[2]), ((bi, b[1]), b[2])]
            lines.append(bench_tuple_workload(args, device, "c2coocsr",
                                              prepared=(spec, ops, (rows, cols),
                                                        f"local Matrix Market files: {names}")))
    else:
        for p in paths:
            t0 = time.perf_counter()
            if args.dims:
                dims = tuple(int(x) for x in args.dims.split(","))
                coords, vals = io.load_frostt(p, dims)
            else:
                big = (2**31 - 1,) * 3
                coords, vals = io.load_frostt(p, big)
                dims = io.frostt_shape(coords)
            a = io.coalesce_coordinates(coords, vals, dims)
            b = io.shift_coordinates(a[0], a[1], dims)
            log(f"parsed {p.name}: shape {dims} nnzA={len(a[1])} nnzB={len(b[1])} "
                f"in {time.perf_counter() - t0:.1f}s")
            ops = [(tuple(np.ascontiguousarray(c[0][:, d]) for d in range(3)), c[1])
                   for c in (a, b)]
            # csf_add and coo3d_add (benchmarks/frostt_tensors_add.py), inner_prod and
            # inner_prod_coo (benchmarks/inner_prod.py) on the same shifted pair
            for w, kernel in (("c5", "csf_add"), ("c5coo", "coo3d_add"),
                              ("c5inner", "inner_prod"), ("c5innercoo", "inner_prod_coo")):
                spec = dict(WORKLOADS[w])
                spec["desc"] = (f"{kernel} f32 of {p.name} (shape {dims}, nnz {len(a[1])}) "
                                f"and its copy shifted by one along every mode")
                data = f"local FROSTT file: {p.name}"
                lines.append(bench_tuple_workload(args, device, w,
                                                  prepared=(spec, ops, dims, data)))
    line = lines[0]
    if len(lines) > 1:
        line["workloads"] = [compact(args.workload, x) for x in lines[1:]]
    return line


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", choices=sorted(WORKLOADS) + ["mtx", "tns"], default="c2")
    ap.add_argument("--files", nargs="*", default=[],
                    help="mtx / tns workloads: local Matrix Market or FROSTT files")
    ap.add_argument("--dims", default="",
                    help="tns workload: I,J,K (default: one past the largest coordinates)")
    ap.add_argument("--only", action="store_true",
                    help="measure --workload alone (no `workloads` list)")
    ap.add_argument("--cpu-budget", type=float, default=12.0,
                    help="seconds of CPU baseline timing (0 disables)")
    ap.add_argument("--extra-cpu-budget", type=float, default=8.0,
                    help="seconds of CPU baseline timing per listed workload")
    ap.add_argument("--extra-steps", type=int, default=20,
                    help="timed steps per listed workload (at most --steps)")
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
        # 5 launches of torch's copy_, then 5 of the library's copy kernel, each 1 GiB in and
        # 1 GiB out: what FETCH_SIZE / WRITE_SIZE read for known bytes
        from nacho_amd import _lib

        lib = _lib.load()
        n = 1 << 28  # 1 GiB of float32
        src = torch.ones(n, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        stream = torch.cuda.current_stream(device).cuda_stream
        for _ in range(5):
            rc = lib.nacho_device_copy(ctypes.c_void_p(dst.data_ptr()),
                                       ctypes.c_void_p(src.data_ptr()), 4 * n,
                                       ctypes.c_void_p(stream))
            if rc != 0:
                raise RuntimeError(_lib.error_string(rc))
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read": 4 * n, "bytes_written": 4 * n,
                          "launches": {"torch copy_": 5, "nacho_device_copy": 5}}))
        return

    if args.workload in ("mtx", "tns"):
        print(json.dumps(bench_files(args, device)), flush=True)
        return
    line = run_workload(args, device, args.workload)
    if args.workload == "c2" and not args.only:
        # The other north-star configurations, measured in the same run: C3 csr_mul, C5 as
        # CSF3 (csf_add) and as COO3 (coo3d_add), then C4 SpGEMM (its cached buffers are
        # released at the end).
        extra = argparse.Namespace(**vars(args))
        extra.steps = max(1, min(args.steps, args.extra_steps))
        extra.warmup = max(1, min(args.warmup, 3))
        extra.cpu_budget = args.extra_cpu_budget if args.cpu_budget > 0 else 0.0
        records = []
        for w in ("c3", "c5", "c5coo", "c4"):
            t0 = time.perf_counter()
            records.append(compact(w, run_workload(extra, device, w)))
            log(f"{w} done in {time.perf_counter() - t0:.1f}s")
            import nacho_amd

            nacho_amd.release_cached_memory()
            torch.cuda.empty_cache()
        line["workloads"] = records
    print(json.dumps(line), flush=True)


def run_workload(args, device, workload):
    if workload == "c4":
        return bench_spgemm(args, device)
    if workload == "c4sssmm":
        return bench_sssmm(args, device)
    if workload in ("c5", "c5coo", "c2coo", "c3coo", "c2dcsr", "c3dcsr", "c5inner",
                    "c5innercoo", "c2coocsr"):
        return bench_tuple_workload(args, device, workload)
    return bench_csr(args, device, workload)


if __name__ == "__main__":
    main()
