#!/usr/bin/env python3
"""VCSR-MC SpMM benchmark on one MI355X.

A step is one SpMM launch of the VCSR-MC kernel over a workload, with A's format, B and C already
resident in HBM.  The default run measures all five workloads at full size, each at its
configured precision and O (segw = 32, tileK = 128):
  1 uniform 4096^2 FP32, O = 128      2 power-law 36,692^2 FP16, O = 128
  3 27-point stencil 100^3 FP32       4 32x32 blocks 262,144^2 FP16, O = 256
  5 R-MAT scale 22 FP16, O = 128
The block workload also runs in FP32 (the case bound by the FP32 matrix cores), as an extra line.
`value` is the power-law workload (the headline configuration) with the reference's C += A.B
semantics; `per_config` holds every workload, in both launch modes (C += A.B, and the additive
C = A.B that never reads C), with its HBM roofline, matrix-core fraction, hipSPARSE FP32/FP16 on
the same GPU in the same run, the row-sample parity check, and the reference's CPU SpMM
(main.cpp:202-207, restated in the oracle) timed on this host on a bounded sample.

Every timed region (K launches after W warm-ups) is preceded by about 30 ms of untimed
launches, so that it measures the GPU's steady state rather than the power transient that
follows an idle period; the launch count is `settle_launches`.  The K timed launches are
captured into one HIP graph after the warm-ups, replayed once untimed (a new graph's first
replay is slower per kernel), then once between the synchronisations (`--eager` enqueues them
one by one instead): the smallest workload's kernel is shorter than the host's enqueue of a
launch.  The reference protocol's single
launches (median of 10 after 3 warm-ups) are taken as the reference takes them.

Prints one JSON line; its last keys, and the last lines of stderr, summarise every workload.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = ("SpMM GFLOP/s (2·nnz·O) at O=128, speedup vs rocSPARSE FP32; "
          "% HBM/MFMA roofline")
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"fp16": 2516.6, "fp32": 157.3}
SEGW, TILEK = 32, 128
HEADLINE = 2
# Sources whose change alters what a launch moves through HBM: the measured traffic in
# profiles/hbm_traffic.json is used only while their hash matches the one it was measured at.
TRAFFIC_SOURCES = ("vcsr_mc_amd/csrc/spmm_kernels.hip", "vcsr_mc_amd/csrc/format_build.hip",
                   "vcsr_mc_amd/csrc/row_groups.hip", "vcsr_mc_amd/csrc/internal.hpp")
PARITY_ROWS = 2000
SETTLE_MS = 30.0  # untimed GPU time before the warm-up launches of every timed region


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--configs", default="1,2,3,4,5,4:fp32",
                   help="workloads to run, comma-separated, each K or K:precision (K:fp32 / "
                        "K:fp16 runs workload K in the other precision); the headline value "
                        "needs 2")
    p.add_argument("--config", type=int, default=None, help="run one workload only")
    p.add_argument("--size", type=int, default=0, help="workload size parameter (0 = full)")
    p.add_argument("--precision", choices=["fp16", "fp32"], default=None)
    p.add_argument("--O", type=int, default=None)
    p.add_argument("--tileK", type=int, default=TILEK)
    p.add_argument("--modes", default="accumulate,overwrite")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-rocsparse", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=24.0,
                   help="CPU-baseline time budget, shared by the workloads")
    p.add_argument("--b-fp32", action="store_true",
                   help="FP16 formats read B in FP32 (the reference's run_vcsr_mc_spmm_gpu path)")
    p.add_argument("--eager", action="store_true",
                   help="enqueue the timed launches one by one instead of replaying them from "
                        "one captured HIP graph")
    p.add_argument("--copy-probe-mib", type=int, default=0,
                   help="also run a plain device copy of this size (PMC traffic calibration)")
    return p.parse_args()


def traffic_source_hash() -> str:
    h = hashlib.sha256()
    for rel in TRAFFIC_SOURCES:
        with open(os.path.join(ROOT, rel), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def measured_traffic(key: str):
    """(HBM bytes per launch, profiled source hash) from rocprofv3 PMC runs, or (None, reason)
    when there is no measurement or it predates the current kernel and layout sources."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if not os.path.exists(path):
        return None, "no profiles/hbm_traffic.json"
    with open(path) as fh:
        d = json.load(fh)
    if d.get("sources_sha256_16") != traffic_source_hash():
        return None, "stale: profiled at other kernel sources"
    e = d.get("launches", {}).get(key)
    if e is None:
        return None, "not profiled"
    return int(e["bytes"]), d["sources_sha256_16"]


def settle(run, stream, ms=SETTLE_MS):
    """Untimed launches for about `ms` of GPU time.  After the GPU has idled (workload
    generation, CPU baseline), a heavy kernel's first few launches run fast, the next few tens
    slower (block FP32, 262,144^2 at O = 256, measured launch by launch after 3 s idle: ~270 us,
    then ~320 us at launches 10-19 and ~288 us at 20-49, then 265 us from launch 50 on); the
    timed region measures the steady state.  Returns the number of launches."""
    import torch
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n, spent = 0, 0.0
    while spent < ms:
        batch = 1 if n == 0 else max(1, min(4096, n))
        e0.record(stream)
        for _ in range(batch):
            run()
        e1.record(stream)
        e1.synchronize()
        spent += e0.elapsed_time(e1)
        n += batch
    return n


def timed_steps(run, steps, warmup, stream, capture=None):
    """A settling phase (see settle), W untimed launches, then K launches bracketed by a
    synchronisation on both sides; the K launches are also bracketed by two HIP events on the
    launch stream.  With `capture` (a function of K returning a callable), the K launches are
    captured into one HIP graph after the warm-ups and the timed region replays it once: the
    same K launches, without the host enqueueing each (the smallest workload's 5 us kernel is
    shorter than one enqueue: 4-6 us per launch through the API, ~14 us in a cold loop's first
    iterations; a graph of 20 launches runs them at 5.5 us each).  The graph is replayed once
    untimed before that: a freshly captured graph's first replay runs each of its kernels
    ~0.75 us slower (uniform 4096^2: 6.1 against 5.35 us per launch, 20 launches), a one-time
    cost of the graph, not of the launches.  Returns (wall ms per step, event ms per step,
    settling launches)."""
    import torch
    settled = settle(run, stream)
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    timed = capture(steps) if capture is not None else None
    if timed is not None:
        timed()  # the graph's first replay, untimed
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    if timed is not None:
        timed()
    else:
        for _ in range(steps):
            run()
    e1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return (t1 - t0) * 1e3 / steps, e0.elapsed_time(e1) / steps, settled


def sub_csr(rp, col, val, rows, np):
    """CSR of the given rows only (same columns)."""
    lens = rp[rows + 1] - rp[rows]
    out = np.zeros(len(rows) + 1, np.int32)
    out[1:] = np.cumsum(lens)
    idx = np.concatenate([np.arange(rp[r], rp[r + 1]) for r in rows]) if out[-1] else \
        np.zeros(0, np.int64)
    return out, col[idx].astype(np.int32), val[idx].astype(np.float32)


def cpu_baseline(A, Bh, O, seconds, oracle, np):
    """The reference's CPU SpMM (main.cpp:202-207: r -> p -> k, double accumulation) on this
    host, through the oracle's restatement: on the whole matrix when one pass is short, else on
    a seeded random sample of rows holding about 2^24 / O nonzeros, repeated for about
    `seconds`; median pass.  1 thread, then every core."""
    if A.nnz * O <= (1 << 26):
        rp, col, val, M, what = A.row_ptr, A.col, A.val, A.M, "the whole workload"
    else:
        rng = np.random.default_rng(7)
        want = (1 << 24) // O
        frac = min(1.0, want / max(A.nnz, 1))
        rows = np.sort(rng.choice(A.M, size=max(1, int(A.M * frac)), replace=False))
        rp, col, val = sub_csr(A.row_ptr, A.col, A.val, rows, np)
        M, what = len(rows), f"a seeded sample of {len(rows)} rows ({int(rp[-1])} nonzeros)"
    nnz = int(rp[-1])
    res = {}
    for threads in (1, os.cpu_count() or 1):
        times, start = [], time.perf_counter()
        while True:
            R = np.zeros((M, O), np.float64)
            t = time.perf_counter()
            oracle.cpu_spmm_f64(rp, col, val, Bh, threads=threads, R=R)
            times.append(time.perf_counter() - t)
            spent = time.perf_counter() - start
            if len(times) >= 3 and spent > seconds / 2:
                break
        res[threads] = (statistics.median(times), len(times))
    flops = 2.0 * nnz * O
    t1, n1 = res[1]
    tall, nall = res[max(res)]
    return ({"value": round(flops / t1 / 1e9, 4), "unit": "GFLOP/s", "cores": 1, "kind": "port",
             "sample": f"{n1} passes over {what} (median pass), double accumulation as "
                       f"main.cpp:202-207"},
            {"value": round(flops / tall / 1e9, 4), "cores": max(res), "passes": nall})


def row_sample_parity(A, Bh, Cgpu, fp32, scale, oracle, np, torch):
    """The launch's C against the oracle on a seeded sample of rows, with the parity norm
    (per row: ||C - C_ref||_1 <= tau * sum |a||b|, tau 1e-5 FP32 / 2e-3 FP16)."""
    rows = np.sort(np.random.default_rng(0).choice(A.M, size=min(A.M, PARITY_ROWS),
                                                   replace=False))
    Cs = Cgpu[torch.from_numpy(rows).to(Cgpu.device)].cpu().numpy().astype(np.float64)
    rp, col, val = sub_csr(A.row_ptr, A.col, A.val, rows, np)
    R, L1 = oracle.spmm_csr(rp, col, val, len(rows), Bh, mode=0 if fp32 else 1, scale=scale)
    err = np.abs(Cs - R).sum(1)
    tau = 1e-5 if fp32 else 2e-3
    return bool(np.all(err <= tau * L1 + 1e-30))


def run_config(cfg, args, stream, want_cpu, cpu_seconds, prec_override=None):
    import numpy as np
    import torch

    import vcsr_mc_amd as vm

    w = vm.WORKLOADS[cfg]
    prec = prec_override or args.precision or w["precision"]
    fp32 = prec == "fp32"
    O = args.O or w["O"]
    dev = torch.device("cuda:0")
    modes = [m for m in args.modes.split(",") if m]
    graphs = []

    t = time.time()
    A = vm.generate(cfg, args.size)
    Bh = vm.dense(A.N, O, seed=vm.SEED_BASE + 100 + cfg, fp16_exact=not fp32)
    log(f"[config {cfg}] {w['name']} size={args.size or 'full'}: {A.M}x{A.N} nnz={A.nnz} "
        f"O={O} {prec} (generated in {time.time() - t:.1f}s)")

    d_rp = torch.from_numpy(A.row_ptr).to(dev)
    d_col = torch.from_numpy(A.col).to(dev)
    d_val = torch.from_numpy(A.val).to(dev)
    dB32 = torch.from_numpy(Bh).to(dev)
    b32 = fp32 or args.b_fp32
    dB = dB32 if b32 else dB32.half()
    C = torch.zeros((A.M, O), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    # GPU format build (the reference's convert + upload, timed apart like its setup_ms)
    t = time.perf_counter()
    fmt = vm.DeviceFormat.from_device_csr(d_rp, d_col, d_val, A.M, A.N, fp32, SEGW)
    torch.cuda.synchronize()
    build_ms = (time.perf_counter() - t) * 1e3
    info = fmt.info()
    log(f"[config {cfg}] format: G={info['num_groups']} items={info['num_items']} "
        f"panels={info['num_panels']} tiles={info['num_chunks']} units={info['num_units']} "
        f"build {build_ms:.1f} ms")

    flops = 2.0 * A.nnz * O
    s_a = 4 if fp32 else 2
    s_b = 4 if b32 else 2
    U = int(np.unique(A.col).size)
    M_ne = int(np.count_nonzero(np.diff(A.row_ptr)))
    # algorithmic bytes: A values and columns, row pointers, each distinct B row once (in the
    # type B is held in), each non-empty C row written once
    bytes_alg = A.nnz * (s_a + 4) + (A.M + 1) * 4 + U * O * s_b + M_ne * O * 4
    # Matrix-core work: the 16 x 32 tiles of the execution layout (each against O columns of B),
    # and, for comparison, the reference's padded 16 x segw groups.
    f_exec = info["num_chunks"] * 2.0 * 16 * 32 * O
    f_pad = info["num_groups"] * 2.0 * 16 * SEGW * O

    out = {"config": cfg, "workload": f"{w['name']}-{A.M}", "M": A.M, "N": A.N, "nnz": A.nnz,
           "O": O, "precision": prec, "B": "fp32" if b32 else "fp16 in HBM",
           "format_build_ms": round(build_ms, 3), "bytes_alg": int(bytes_alg),
           "layout": {k: info[k] for k in ("num_panels", "num_chunks", "num_units", "num_heavy",
                                           "num_split_panels", "num_dense", "row_grouped",
                                           "num_row_step_batches")}}
    full = args.size == 0 and O == w["O"] and args.tileK == TILEK and not args.b_fp32
    oracle = None
    if want_cpu:
        import oracle as oracle_mod
        oracle_mod.build()
        oracle = oracle_mod

    for mode in modes:
        ow = mode == "overwrite"

        # the timed launches go through a pre-bound launcher: the checks of fmt.spmm take
        # longer than the smallest workload's kernel, and the loop must keep the GPU fed
        step = fmt.launcher(dB, C, tileK=args.tileK, O=O, stream=stream, overwrite=ow)

        # reference protocol: median of 10 event-timed single launches after 3 warm-ups, C
        # zeroed outside the timing (main.cpp:239-298)
        single = []
        for i in range(13):
            C.zero_()
            ms = fmt.spmm(dB, C, tileK=args.tileK, O=O, stream=stream, timed=True, overwrite=ow)
            if i >= 3:
                single.append(ms)
        ms_single = statistics.median(single)
        parity = (row_sample_parity(A, Bh, C, fp32, info["scale"], oracle, np, torch)
                  if oracle is not None else None)

        def capture(k, ow=ow):
            """The k timed launches as one HIP graph, replayed on the launch stream (the
            launch enqueues kernels only: no allocation, no memset)."""
            graph = torch.cuda.CUDAGraph()
            cap = torch.cuda.Stream()
            cap.wait_stream(stream)
            with torch.cuda.graph(graph, stream=cap):
                for _ in range(k):
                    fmt.spmm(dB, C, tileK=args.tileK, O=O, stream=cap, overwrite=ow)
            stream.wait_stream(cap)
            graphs.append(graph)  # kept until the workload's buffers are freed
            return graph.replay

        C.zero_()
        ms_per_step, kernel_ms, settled = timed_steps(step, args.steps, args.warmup, stream,
                                                      None if args.eager else capture)
        achieved = bytes_alg / (kernel_ms * 1e-3) / 1e9
        traffic, stamp = measured_traffic(f"config{cfg}-{prec}-{mode}") if full else \
            (None, "measured at the full workload only")
        # what this launch's schedule cannot avoid moving, if each XCD's L2 kept everything
        # its work-groups touched: B per XCD row part, the layout per O tile, C once (twice
        # accumulating)
        floor = fmt.traffic_floor(O, tileK=args.tileK, b_f16=not b32, overwrite=ow)
        floor_rate = floor["total"] / (kernel_ms * 1e-3) / 1e9
        mfma_tf = f_exec / (kernel_ms * 1e-3) / 1e12
        ref_tf = f_pad / (kernel_ms * 1e-3) / 1e12
        out[mode] = {
            "ms_per_step": round(ms_per_step, 6),
            "settle_launches": settled,
            "timed_launches": "enqueued one by one" if args.eager else "one HIP graph of K",
            "gflops": round(flops / (ms_per_step * 1e-3) / 1e9, 2),
            "kernel_ms": round(kernel_ms, 6),
            "kernel_gflops": round(flops / (kernel_ms * 1e-3) / 1e9, 2),
            "single_launch_median_ms": round(ms_single, 6),
            "single_launch_gflops": round(flops / (ms_single * 1e-3) / 1e9, 2),
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                         "traffic": traffic, "traffic_source": stamp,
                         "floor_bytes": int(floor["total"]),
                         "floor_frac": round(floor_rate / HBM_PEAK_GBS, 4),
                         "frac_ceiling": round(bytes_alg / floor["total"], 4),
                         "floor": {k: floor[k] for k in ("b_bytes", "b_once_bytes", "a_bytes",
                                                         "c_bytes", "convert_bytes",
                                                         "o_tile_width", "row_parts")}},
            "mfma": {"executed_tflops": round(mfma_tf, 2), "peak": MFMA_PEAK_TFLOPS[prec],
                     "frac": round(mfma_tf / MFMA_PEAK_TFLOPS[prec], 5),
                     "ref_padded_tflops": round(ref_tf, 2),
                     "ref_padded_frac": round(ref_tf / MFMA_PEAK_TFLOPS[prec], 5)},
            "parity_row_sample": parity,
        }
        log(f"[config {cfg}] {mode}: {kernel_ms * 1e3:.2f} us/launch back to back, single "
            f"{ms_single * 1e3:.2f} us, {achieved / HBM_PEAK_GBS:.3f} of HBM peak "
            f"(floor {floor['total'] / 1e6:.1f} MB: {floor_rate / HBM_PEAK_GBS:.3f}), "
            f"parity {parity}")

    if not args.no_rocsparse:
        rs = {}
        for label, vf16, bf16 in (("fp32", False, False), ("fp16", True, True)):
            vv = d_val.half() if vf16 else d_val
            BB = dB32.half() if bf16 else dB32
            alpha = 1.0 if not vf16 else info["scale"]
            Cr = torch.zeros_like(C)
            times = []
            for i in range(13):
                ms, setup = vm.rocsparse_spmm(A.M, A.N, d_rp, d_col, vv, BB, Cr, alpha=alpha,
                                              stream=stream)
                if i >= 3:
                    times.append(ms)
            med = statistics.median(times)
            rs[label] = {"ms_median": round(med, 6), "gflops": round(flops / (med * 1e-3) / 1e9, 2),
                         "setup_ms": round(setup, 3)}
            del Cr
        vm.bench_lib().vcsrmc_rocsparse_release()
        out["rocsparse"] = rs
        for mode in modes:
            ours = out[mode]["single_launch_median_ms"]
            out[mode]["speedup_vs_rocsparse_fp32"] = round(rs["fp32"]["ms_median"] / ours, 3)
            out[mode]["speedup_vs_rocsparse_fp16"] = round(rs["fp16"]["ms_median"] / ours, 3)

    if want_cpu:
        out["cpu_baseline"], out["cpu_baseline_all_cores"] = cpu_baseline(
            A, Bh, O, cpu_seconds, oracle, np)
        log(f"[config {cfg}] CPU baseline {out['cpu_baseline']['value']} GFLOP/s (1 core)")

    del graphs[:]
    fmt.close()
    del C, dB, dB32, d_rp, d_col, d_val
    torch.cuda.empty_cache()
    return out


def vm_precision(cfg):
    import vcsr_mc_amd as vm
    return vm.WORKLOADS[cfg]["precision"]


def geomean(xs):
    return math.exp(sum(math.log(x) for x in xs) / len(xs)) if xs else None


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU (--gpus 1): the VCSR-MC path runs on one device; "
              "splitting it across GPUs by output columns is not implemented.", file=sys.stderr)
        sys.exit(2)

    import torch

    spec = [str(args.config)] if args.config else [c for c in args.configs.split(",") if c]
    configs = []
    for c in spec:
        k, _, pr = c.partition(":")
        if pr not in ("", "fp16", "fp32"):
            print(f"--configs: unknown precision in {c}", file=sys.stderr)
            sys.exit(2)
        configs.append((int(k), pr or None))
    modes = [m for m in args.modes.split(",") if m]
    if any(m not in ("accumulate", "overwrite") for m in modes) or not modes:
        print("--modes takes accumulate and/or overwrite", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()
    want_cpu = not args.no_cpu

    per = []
    for cfg, pr in configs:
        per.append(run_config(cfg, args, stream, want_cpu, args.cpu_seconds / len(configs), pr))

    # each workload at its configured precision; the others are extra lines of per_config
    configured = [p for p in per if p["precision"] == vm_precision(p["config"])]
    head = next((p for p in configured if p["config"] == HEADLINE), per[0])
    hm = "accumulate" if "accumulate" in modes else modes[0]
    h = head[hm]
    out = {
        "metric": METRIC,
        "value": h["gflops"],
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms_before_warmup": SETTLE_MS,
        "timed_launches": ("enqueued one by one" if args.eager else
                           "one HIP graph of K launches, its first replay untimed"),
        "ms_per_step": h["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if head["precision"] == "fp32" else "f16",
        "data": "synthetic",
        "config": {"workload": f"{head['workload']} (config {head['config']})", "M": head["M"],
                   "N": head["N"], "nnz": head["nnz"], "O": head["O"], "segw": SEGW,
                   "tileK": args.tileK, "precision": head["precision"], "B": head["B"],
                   "accumulate": "C += A.B" if hm == "accumulate" else "C = A.B"},
        "kernel_ms": h["kernel_ms"],
        "kernel_ms_single_launch_median": h["single_launch_median_ms"],
        "roofline": dict(h["roofline"], bytes_alg=head["bytes_alg"]),
        "mfma": h["mfma"],
        "parity_row_sample": h["parity_row_sample"],
    }
    if "rocsparse" in head:
        out["rocsparse"] = head["rocsparse"]
        out["speedup_vs_rocsparse_fp32"] = h["speedup_vs_rocsparse_fp32"]
    if "cpu_baseline" in head:
        out["cpu_baseline"] = head["cpu_baseline"]
        out["cpu_baseline_all_cores"] = head["cpu_baseline_all_cores"]
        try:
            out["cpu_model"] = [l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo")
                                if l.startswith("model name")][0]
        except Exception:
            out["cpu_model"] = "unknown"
    # the target: geomean over workloads 1-4 of rocSPARSE FP32 time / ours, each at its
    # configured precision, reference protocol (median single launch)
    if not args.no_rocsparse:
        for mode in modes:
            sp = [p[mode]["speedup_vs_rocsparse_fp32"] for p in configured
                  if p["config"] in (1, 2, 3, 4)]
            if len(sp) == 4:
                out[f"speedup_vs_rocsparse_fp32_geomean_1_4_{mode}"] = round(geomean(sp), 3)
    out["per_config"] = per
    # The target in a few lines, last in the JSON line and in stderr (a reader of either tail
    # finds it): per workload and mode, our single-launch median, rocSPARSE FP32's, the ratio,
    # the HBM fraction, measured traffic and the schedule's floor over the algorithmic bytes.
    summary = []
    for p in per:
        for mode in modes:
            m = p[mode]
            rf = m["roofline"]
            row = {"w": f"{p['config']}:{p['precision']}", "mode": mode[:3],
                   "us": round(m["single_launch_median_ms"] * 1e3, 2),
                   "frac": rf["frac"], "floor/alg": round(rf["floor_bytes"] / p["bytes_alg"], 2),
                   "traffic/alg": (round(rf["traffic"] / p["bytes_alg"], 2)
                                   if rf["traffic"] else None)}
            if "rocsparse" in p:
                row["rs32_us"] = round(p["rocsparse"]["fp32"]["ms_median"] * 1e3, 2)
                row["x"] = m["speedup_vs_rocsparse_fp32"]
            summary.append(row)
    out["summary"] = summary
    for mode in modes:
        k = f"speedup_vs_rocsparse_fp32_geomean_1_4_{mode}"
        if k in out:
            out[k] = out.pop(k)  # moved after per_config
    log("[summary] workload:precision mode | ours us | rocSPARSE FP32 us | speedup | HBM frac "
        "| traffic/alg | floor/alg  (single-launch medians)")
    for row in summary:
        log("[summary] {w} {mode} | {us} | {rs} | {x} | {frac} | {t} | {f}".format(
            rs=row.get("rs32_us"), x=row.get("x"), t=row["traffic/alg"], f=row["floor/alg"],
            **{k: row[k] for k in ("w", "mode", "us", "frac")}))
    for mode in modes:
        k = f"speedup_vs_rocsparse_fp32_geomean_1_4_{mode}"
        if k in out:
            log(f"[summary] geomean speedup vs rocSPARSE FP32, workloads 1-4 at their "
                f"configured precision, {mode}: {out[k]}")

    if args.copy_probe_mib:
        # a plain copy of known size: reads and writes copy_probe_mib MiB once
        nelem = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(nelem, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        out["copy_probe_bytes"] = nelem * 4

    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
