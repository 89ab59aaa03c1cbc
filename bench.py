#!/usr/bin/env python3
"""VCSR-MC SpMM benchmark on one MI355X.

A step is one C += A.B launch of the VCSR-MC kernel over the workload, with A's format, B and C
already resident in HBM.  Default workload: the power-law graph matrix 36,692 x 36,692 (~352k
nnz, FP16 A and B, FP32 C), O = 128, segw = 32, tileK = 128 -- the configuration the headline
metric is quoted on.  `--config k` picks another workload (1 uniform FP32, 3 stencil FP32,
4 block FP16 at O = 256, 5 R-MAT FP16).

Prints one JSON line: GFLOP/s = 2 nnz O / t, the HBM roofline of the kernel (algorithmic bytes
nnz (s_A + 4) + (M + 1) 4 + U O s_B + M_ne O 4 over the event-timed kernel duration), the MFMA
fraction of the padded reference tiles, hipSPARSE FP32/FP16 on the same GPU in the same run,
and the reference's CPU SpMM (main.cpp:202-207, restated in the oracle) timed on this host.
"""
from __future__ import annotations

import argparse
import json
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


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--config", type=int, default=2)
    p.add_argument("--size", type=int, default=0, help="workload size parameter (0 = full)")
    p.add_argument("--precision", choices=["fp16", "fp32"], default=None)
    p.add_argument("--O", type=int, default=None)
    p.add_argument("--tileK", type=int, default=TILEK)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-rocsparse", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--b-fp32", action="store_true",
                   help="FP16 format with B left in FP32 (the reference's run_vcsr_mc_spmm_gpu path)")
    p.add_argument("--graph", action="store_true",
                   help="replay the timed steps from a captured HIP graph")
    p.add_argument("--copy-probe-mib", type=int, default=0,
                   help="also run a plain device copy of this size (PMC traffic calibration)")
    return p.parse_args()


def traffic_from_profiles(workload: str):
    """HBM bytes per launch measured with rocprofv3 PMC counters (profiles/*.json)."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as fh:
            return json.load(fh).get(workload)
    except Exception:
        return None


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU (--gpus 1): the VCSR-MC path runs on one device; "
              "splitting it across GPUs by output columns is not implemented.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import vcsr_mc_amd as vm

    cfg = args.config
    w = vm.WORKLOADS[cfg]
    prec = args.precision or w["precision"]
    fp32 = prec == "fp32"
    O = args.O or w["O"]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()

    t = time.time()
    A = vm.generate(cfg, args.size)
    log(f"workload {w['name']} size={args.size or 'full'}: {A.M}x{A.N} nnz={A.nnz} "
        f"({time.time() - t:.1f}s)")
    Bh = vm.dense(A.N, O, seed=vm.SEED_BASE + 100 + cfg, fp16_exact=not fp32)

    d_rp = torch.from_numpy(A.row_ptr).to(dev)
    d_col = torch.from_numpy(A.col).to(dev)
    d_val = torch.from_numpy(A.val).to(dev)
    dB32 = torch.from_numpy(Bh).to(dev)
    dB = dB32 if (fp32 or args.b_fp32) else dB32.half()
    C = torch.zeros((A.M, O), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    # GPU format build (the reference's convert + upload, timed separately like setup_ms)
    t = time.perf_counter()
    fmt = vm.DeviceFormat.from_device_csr(d_rp, d_col, d_val, A.M, A.N, fp32, SEGW)
    torch.cuda.synchronize()
    build_ms = (time.perf_counter() - t) * 1e3
    info = fmt.info()
    log(f"format: G={info['num_groups']} items={info['num_items']} panels={info['num_panels']} "
        f"tiles={info['num_chunks']} units={info['num_units']} build {build_ms:.1f} ms")

    def step():
        fmt.spmm(dB, C, tileK=args.tileK, O=O, stream=stream)

    # reference protocol: median of single event-timed launches (C zeroed outside the timing)
    for _ in range(3):
        C.zero_()
        fmt.spmm(dB, C, tileK=args.tileK, O=O, stream=stream, timed=True)
    single = []
    for _ in range(10):
        C.zero_()
        single.append(fmt.spmm(dB, C, tileK=args.tileK, O=O, stream=stream, timed=True))
    ms_single_median = statistics.median(single)

    graph = None
    if args.graph:
        # captured on a side stream (capture is refused on the default one), replayed on
        # `stream`, where the timing events are recorded
        graph = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(stream)
        with torch.cuda.graph(graph, stream=cap):
            fmt.spmm(dB, C, tileK=args.tileK, O=O, stream=cap)
        stream.wait_stream(cap)
        run = graph.replay
    else:
        run = step

    C.zero_()
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    kernel_ms = e0.elapsed_time(e1) / args.steps

    flops = 2.0 * A.nnz * O
    gflops = flops / (ms_per_step * 1e-3) / 1e9

    # algorithmic bytes: A values and columns, row pointers, each distinct B row once (in the
    # element type B is held in), each non-empty C row once
    s_a = 4 if fp32 else 2
    s_b = 4 if (fp32 or args.b_fp32) else 2
    U = int(np.unique(A.col).size)
    M_ne = int(np.count_nonzero(np.diff(A.row_ptr)))
    bytes_alg = A.nnz * (s_a + 4) + (A.M + 1) * 4 + U * O * s_b + M_ne * O * 4
    achieved_gbs = bytes_alg / (kernel_ms * 1e-3) / 1e9
    f_pad = info["num_groups"] * 2.0 * 16 * SEGW * O
    mfma_tflops = f_pad / (kernel_ms * 1e-3) / 1e12

    out = {
        "metric": METRIC,
        "value": round(gflops, 2),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if fp32 else "f16",
        "data": "synthetic",
        "config": {"workload": f"{w['name']}-{A.M} (config {cfg})", "M": A.M, "N": A.N,
                   "nnz": A.nnz, "O": O, "segw": SEGW, "tileK": args.tileK,
                   "precision": prec, "B": "fp32" if (fp32 or args.b_fp32) else "fp16 in HBM",
                   "accumulate": "C += A.B"},
        "kernel_ms": round(kernel_ms, 6),
        "kernel_ms_single_launch_median": round(ms_single_median, 6),
        "gflops_single_launch_median": round(flops / (ms_single_median * 1e-3) / 1e9, 2),
        "format_build_ms": round(build_ms, 3),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
            # measured for the full workload at its O and tileK 128 (profiles/); other runs: null
            "traffic": (traffic_from_profiles(f"config{cfg}-{prec}")
                        if args.size == 0 and O == w["O"] and args.tileK == TILEK
                        and not args.b_fp32 else None),
            "bytes_alg": int(bytes_alg),
        },
        "mfma": {"padded_tflops": round(mfma_tflops, 2), "peak": MFMA_PEAK_TFLOPS[prec],
                 "frac": round(mfma_tflops / MFMA_PEAK_TFLOPS[prec], 5),
                 "padded_flop": f_pad},
    }

    if not args.no_rocsparse:
        rs_out = {}
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
            rs_out[label] = {"ms_median": round(med, 6),
                             "gflops": round(flops / (med * 1e-3) / 1e9, 2),
                             "setup_ms": round(setup, 3)}
        vm.bench_lib().vcsrmc_rocsparse_release()
        out["rocsparse"] = rs_out
        out["speedup_vs_rocsparse_fp32"] = round(rs_out["fp32"]["ms_median"] / ms_single_median, 3)
        out["speedup_vs_rocsparse_fp16"] = round(rs_out["fp16"]["ms_median"] / ms_single_median, 3)

    if not args.no_cpu:
        # The CPU leg runs the oracle's restatement of the reference's CPU SpMM.  First, as a
        # check (the numbers above are reported only beside it): one launch, from C = 0,
        # against that product on a 2000-row sample, with the parity norm.
        import oracle
        oracle.build()
        C.zero_()
        step()
        torch.cuda.synchronize()
        rs = np.random.default_rng(0).choice(A.M, size=min(A.M, 2000), replace=False)
        rs.sort()
        lens = A.row_ptr[rs + 1] - A.row_ptr[rs]
        srp = np.zeros(len(rs) + 1, np.int32)
        srp[1:] = np.cumsum(lens)
        idx = np.concatenate([np.arange(A.row_ptr[r], A.row_ptr[r + 1]) for r in rs])
        R, L1 = oracle.spmm_csr(srp, A.col[idx], A.val[idx], len(rs), Bh,
                                mode=0 if fp32 else 1, scale=info["scale"])
        err = np.abs(C.cpu().numpy()[rs].astype(np.float64) - R).sum(1)
        tau = 1e-5 if fp32 else 2e-3
        out["parity_row_sample"] = bool(np.all(err <= tau * L1 + 1e-30))

        # The reference's CPU SpMM (main.cpp:202-207, double accumulation) on this host: full
        # passes over the whole matrix repeated for about --cpu-seconds, median pass.
        def cpu_pass(threads):
            Rb = np.zeros((A.M, O), np.float64)
            t = time.perf_counter()
            oracle.cpu_spmm_f64(A.row_ptr, A.col, A.val, Bh, threads=threads, R=Rb)
            return time.perf_counter() - t
        res = {}
        for threads in (1, os.cpu_count() or 1):
            times, start = [], time.perf_counter()
            while time.perf_counter() - start < args.cpu_seconds / 2 or len(times) < 3:
                times.append(cpu_pass(threads))
                if len(times) >= 3 and time.perf_counter() - start > args.cpu_seconds:
                    break
            res[threads] = (statistics.median(times), len(times))
        t1s, n1 = res[1]
        out["cpu_baseline"] = {
            "value": round(flops / t1s / 1e9, 4), "unit": "GFLOP/s", "cores": 1, "kind": "port",
            "sample": f"{n1} full passes over the whole workload (median), "
                      f"double accumulation as main.cpp:202-207",
        }
        tall, nall = res[max(res)]
        out["cpu_baseline_all_cores"] = {"value": round(flops / tall / 1e9, 4), "cores": max(res),
                                         "passes": nall}
        try:
            model = [l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo")
                     if l.startswith("model name")][0]
        except Exception:
            model = "unknown"
        out["cpu_model"] = model

    if args.copy_probe_mib:
        # a plain copy of known size: reads and writes copy_probe_mib MiB once
        nelem = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(nelem, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        out["copy_probe_bytes"] = nelem * 4

    fmt.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
