"""Times the reference's own VCSR-MC kernels against this library's, with the reference's driver
and protocol on both sides (run on a machine with an MI355X; not a pytest module).

* oracle/_ref/spmm_vcsr_ref:    the reference's src/main.cpp, src/kernels.cu and src/vcsr_mc.cu,
                                built as-is for gfx950 (`make -C oracle ref`);
* oracle/_ref/spmm_vcsr_dropin: the same main.cpp and kernels.cu against this repository's
                                include/, linked with libvcsrmc.so.
Both read the same Matrix Market file (the workload written by `spmm_vcsr --gen K
--write-mtx`) and run `--algo vcsr_mc[,vcsr_mc_fp32] --segw 32 --tileK 128 --stat median`
(median of 10 event-timed single launches after 3 warm-ups, C zeroed before each,
src/main.cpp:239-298), with FP32 B as the reference's API takes it and its hipSPARSE check.

    python tests/ref_kernel_timing.py [--configs 1,2,3,4] [--both-precisions] [--out FILE]

Prints a table and the geomean of the speedups over the workloads run at their configured
precision."""
import argparse
import csv
import io
import math
import os
import subprocess
import sys
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.path.join(ROOT, "oracle", "_ref", "spmm_vcsr_ref")
DROPIN = os.path.join(ROOT, "oracle", "_ref", "spmm_vcsr_dropin")
DRIVER = os.path.join(ROOT, "vcsr_mc_amd", "spmm_vcsr")
WORKLOADS = {1: ("uniform 4096^2", "vcsr_mc_fp32", 128), 2: ("power-law 36,692^2", "vcsr_mc", 128),
             3: ("stencil 100^3", "vcsr_mc_fp32", 128), 4: ("block 32x32, 262,144^2", "vcsr_mc", 256),
             5: ("R-MAT scale 22", "vcsr_mc", 128)}


def timed(binary, mtx, algos, O):
    args = [binary, "--mtx", mtx, "--O", str(O), "--segw", "32", "--tileK", "128", "--repeat",
            "10", "--warmup", "3", "--stat", "median", "--csv", "--bdist", "uniform",
            "--algo", ",".join(algos)]
    print("[run]", " ".join(os.path.basename(a) for a in args[:1]) , *args[1:], flush=True)
    r = subprocess.run(args, capture_output=True, text=True, timeout=1200)
    if r.returncode != 0:
        sys.exit(f"{os.path.basename(binary)} failed: {r.stderr[-2000:]}")
    return {row["algo"]: row for row in csv.DictReader(io.StringIO(r.stdout))}


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--configs", default="1,2,3,4")
    p.add_argument("--both-precisions", action="store_true")
    p.add_argument("--out", default=None)
    a = p.parse_args()
    for b in (REF, DROPIN, DRIVER):
        if not os.path.exists(b):
            sys.exit(f"{b} is not built")
    lines = ["| workload | kernel | reference kernel us | this library us | speedup | validation |",
             "|---|---|---|---|---|---|"]
    speedups = []
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR", "/tmp")) as tmp:
        for cfg in [int(c) for c in a.configs.split(",")]:
            name, algo, O = WORKLOADS[cfg]
            mtx = os.path.join(tmp, f"w{cfg}.mtx")
            print(f"[workload {cfg}] writing {name}", flush=True)
            subprocess.run([DRIVER, "--gen", str(cfg), "--write-mtx", mtx], check=True)
            algos = ["vcsr_mc", "vcsr_mc_fp32"] if a.both_precisions else [algo]
            ref = timed(REF, mtx, algos, O)
            ours = timed(DROPIN, mtx, algos, O)
            for k in algos:
                r_us, o_us = float(ref[k]["ms"]) * 1e3, float(ours[k]["ms"]) * 1e3
                lines.append(f"| {name} | {k} | {r_us:.1f} | {o_us:.1f} | {r_us / o_us:.2f}x | "
                             f"{ref[k]['validation']} / {ours[k]['validation']} |")
                if k == algo and cfg <= 4:
                    speedups.append(r_us / o_us)
            os.remove(mtx)
            print("\n".join(lines), flush=True)
    if speedups:
        g = math.exp(sum(math.log(s) for s in speedups) / len(speedups))
        lines.append(f"\nGeomean over the configured workloads 1-4 run: {g:.2f}x")
    text = "\n".join(lines) + "\n"
    print(text)
    if a.out:
        with open(a.out, "w") as fh:
            fh.write(text)


if __name__ == "__main__":
    main()
