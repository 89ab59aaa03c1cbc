"""Corpus sweep protocol for the spmm_vcsr driver: run, rerun noisy matrices, tabulate.

The same protocol as the reference's harness (bench200/run200.py, rerun_noisy.py, analyze.py,
orig_table.py, run.sh of MuuSeoTia/VCSR_MC), for a corpus of Matrix Market files supplied
locally (nothing is downloaded):

* run: one fresh driver process per (matrix, algorithm, repetition), each with
  ``--mtx --algo --csv`` plus the extra arguments; rows are tagged with the corpus nnz and the
  repetition and written to one CSV with the reference's columns (run200.py:24-27).  A failing or
  timed-out process is reported and skipped (run200.py:42-56).
* rerun: a matrix is noisy when, for some algorithm, its slowest repetition is more than 2x its
  fastest; noisy matrices are run again with 5 repetitions and their rows replaced, the original
  CSV kept as ``<name>_raw.csv`` (rerun_noisy.py:2-8, 24-59).
* table: per (matrix, algorithm) the median over repetitions (analyze.py:7-10, 32), speedup =
  t_rocsparse / t_kernel, and per kernel the geometric mean, geometric standard deviation
  exp(sigma of log speedup), median, min, max, wins and the largest rel_l2, for the mean and the
  median launch time columns, pooled over widths O when several CSVs are given
  (orig_table.py:17-40, analyze.py:38-45).

Usage::

    python -m vcsr_mc_amd.sweep run   BINARY CORPUS.csv MTXDIR OUT.csv
    python -m vcsr_mc_amd.sweep rerun BINARY CORPUS.csv MTXDIR RESULTS.csv [...]
    python -m vcsr_mc_amd.sweep table RESULTS.csv [...]
    python -m vcsr_mc_amd.sweep all   --corpus CORPUS.csv --mtx-dir MTXDIR [--tag T] [--O 128 ...]

``ALGOS``, ``REPS`` and ``EXTRA`` are read from the environment when the options are not given,
like the reference's scripts.
"""
from __future__ import annotations

import argparse
import collections
import csv
import io
import math
import os
import shlex
import shutil
import socket
import subprocess
import sys
import time
from pathlib import Path

FIELDS = ["gpu", "sm", "mtx", "O", "segw", "bundle", "tileK", "repeat", "algo", "ms", "gflops",
          "validation", "rel_l2", "setup_ms", "nnz", "rep", "ms_mean", "ms_median", "convert_ms",
          "upload_ms"]
DEFAULT_ALGOS = ["rocsparse", "rocsparse_fp16", "vcsr_mc", "vcsr_mc_fp32"]
BASE = "rocsparse"
KERNELS = ["vcsr_mc", "vcsr_mc_fp32"]
SPREAD, RERUN_REPS = 2.0, 5
DRIVER = Path(__file__).resolve().parent / "spmm_vcsr"


def _env_list(name: str, default: list[str]) -> list[str]:
    v = os.environ.get(name)
    return v.replace(",", " ").split() if v else list(default)


def matrix_name(mtx: str) -> str:
    base = mtx.replace("\\", "/").split("/")[-1]
    return base[:-4] if base.endswith(".mtx") else base


# ---- statistics (analyze.py:7-10, 38-45) ------------------------------------------------
def median(v):
    v = sorted(v)
    n = len(v)
    if n == 0:
        raise ValueError("median of nothing")
    return v[n // 2] if n % 2 else 0.5 * (v[n // 2 - 1] + v[n // 2])


def geo_gstd(vals):
    """Geometric mean and geometric standard deviation exp(sigma of log x), sigma over n."""
    if not vals:
        return float("nan"), float("nan")
    lg = [math.log(x) for x in vals]
    mu = sum(lg) / len(lg)
    sd = math.sqrt(sum((x - mu) ** 2 for x in lg) / len(lg))
    return math.exp(mu), math.exp(sd)


def load(path, col: str = "ms"):
    """Per (matrix, algo): median of `col` over its rows, GFLOP/s at that time, largest rel_l2.

    GFLOP/s for another timing column is recomputed from the row's FLOP count
    (gflops x ms), which every row of a matrix shares.  Returns (gflops, ms, rel_l2, nnz), each a
    dict matrix -> algo -> value (nnz: matrix -> int)."""
    times = collections.defaultdict(lambda: collections.defaultdict(list))
    errs = collections.defaultdict(lambda: collections.defaultdict(list))
    mflop, nnz = {}, {}
    with open(path, newline="") as fh:
        for r in csv.DictReader(fh):
            m = matrix_name(r["mtx"])
            t = float(r[col])
            times[m][r["algo"]].append(t)
            errs[m][r["algo"]].append(float(r["rel_l2"]))
            if float(r["ms"]) > 0:
                mflop[m] = float(r["gflops"]) * float(r["ms"])
            nnz[m] = int(r["nnz"]) if r.get("nnz") else 0
    g, t, e = (collections.defaultdict(dict) for _ in range(3))
    for m in times:
        for a, v in times[m].items():
            t[m][a] = median(v)
            g[m][a] = mflop.get(m, 0.0) / t[m][a] if t[m][a] > 0 else 0.0
            e[m][a] = max(errs[m][a])
    return g, t, e, nnz


# ---- run (run200.py) ----------------------------------------------------------------------
def run(binary, corpus, mtxdir, out, algos=None, reps=None, extra=None, timeout=300, log=None):
    """One process per (matrix, algo, rep); returns the number of rows written."""
    algos = algos or _env_list("ALGOS", DEFAULT_ALGOS)
    reps = reps if reps is not None else int(os.environ.get("REPS", "1"))
    extra = extra if extra is not None else shlex.split(os.environ.get("EXTRA", ""))
    log = log or sys.stderr
    rows = 0
    with open(out, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=FIELDS, extrasaction="ignore")
        w.writeheader()
        with open(corpus, newline="") as cf:
            entries = list(csv.DictReader(cf))
        for m in entries:
            mtx = Path(mtxdir) / f"{m['name']}.mtx"
            if not mtx.is_file():
                print(f"missing {mtx}", file=log)
                continue
            for rep in range(reps):
                for algo in algos:
                    cmd = [str(binary), "--mtx", str(mtx), "--algo", algo, "--csv"] + list(extra)
                    try:
                        r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
                    except subprocess.TimeoutExpired:
                        print(f"timeout {m['name']} {algo} rep{rep}", file=log)
                        continue
                    if r.returncode != 0:
                        err = (r.stderr or "").strip().splitlines()
                        print(f"fail {m['name']} {algo} rep{rep}: {err[-1] if err else r.returncode}",
                              file=log)
                        continue
                    for row in csv.DictReader(io.StringIO(r.stdout)):
                        row["nnz"] = m.get("nnz", "")
                        row["rep"] = rep
                        w.writerow(row)
                        rows += 1
                    fh.flush()
            print(m["name"], file=log, flush=True)
    return rows


# ---- rerun (rerun_noisy.py) -------------------------------------------------------------
def noisy_matrices(rows, spread: float = SPREAD):
    ms = collections.defaultdict(list)
    for r in rows:
        ms[(matrix_name(r["mtx"]), r["algo"])].append(float(r["ms"]))
    return sorted({m for (m, _), v in ms.items() if min(v) > 0 and max(v) / min(v) > spread})


def _protocol_extra(extra, O, tileK):
    """The sweep's extra arguments with --O / --tileK taken from the results file."""
    rest, toks = [], list(extra)
    while toks:
        t = toks.pop(0)
        if t in ("--O", "--tileK"):
            if toks:
                toks.pop(0)
        else:
            rest.append(t)
    return ["--O", str(O), "--tileK", str(tileK)] + rest


def rerun_noisy(binary, corpus, mtxdir, paths, algos=None, extra=None, reps=RERUN_REPS,
                spread=SPREAD, log=None):
    """Reruns the noisy matrices of each results CSV in place; returns {path: [names]}."""
    log = log or sys.stdout
    algos = algos or _env_list("ALGOS", ["rocsparse", "vcsr_mc"])
    extra = extra if extra is not None else shlex.split(
        os.environ.get("EXTRA", "--repeat 10 --warmup 0 --stat median"))
    done = {}
    for path in map(Path, paths):
        raw = path.with_name(path.stem + "_raw.csv")
        if not raw.exists():
            shutil.copy(path, raw)
        with raw.open(newline="") as fh:
            rows = list(csv.DictReader(fh))
        noisy = noisy_matrices(rows, spread)
        done[str(path)] = noisy
        if not rows:
            continue
        O, tk = rows[0]["O"], rows[0]["tileK"]
        print(f"{path.name}: O={O}, {len(noisy)} noisy: {' '.join(noisy)}", file=log, flush=True)
        if not noisy:
            continue
        sub = path.with_name(path.stem + "_rerun_corpus.csv")
        with open(corpus, newline="") as cf, sub.open("w", newline="") as fh:
            reader = csv.DictReader(cf)
            w = csv.DictWriter(fh, fieldnames=reader.fieldnames)
            w.writeheader()
            w.writerows(m for m in reader if m["name"] in noisy)
        out = path.with_name(path.stem + "_rerun.csv")
        run(binary, sub, mtxdir, out, algos=algos, reps=reps, extra=_protocol_extra(extra, O, tk))
        with out.open(newline="") as fh:
            new = list(csv.DictReader(fh))
        with path.open("w", newline="") as fh:
            w = csv.DictWriter(fh, fieldnames=list(rows[0].keys()), extrasaction="ignore")
            w.writeheader()
            w.writerows(r for r in rows if matrix_name(r["mtx"]) not in noisy)
            w.writerows(new)
        sub.unlink()
        print(f"  replaced with {len(new)} rows from {reps} reps -> {path.name}", file=log,
              flush=True)
    return done


# ---- table (orig_table.py) ----------------------------------------------------------------
def speedups(path, col, kernel, base=BASE):
    _, t, e, _ = load(path, col)
    sp = [t[m][base] / t[m][kernel] for m in t
          if t[m].get(base, 0) > 0 and t[m].get(kernel, 0) > 0]
    err = max((e[m][kernel] for m in e if kernel in e[m]), default=float("nan"))
    return sp, err


def summary(sp):
    gm, gs = geo_gstd(sp)
    return dict(n=len(sp), geomean=gm, gstd=gs, median=median(sp), min=min(sp), max=max(sp),
                wins=sum(s > 1 for s in sp))


def table(paths, kernels=KERNELS, base=BASE, out=None) -> dict:
    """Prints the speedup table; returns {(col, O or 'all', kernel): summary}."""
    out = out or sys.stdout
    res = {}
    for col, what in (("ms_mean", "MEAN of the timed launches"),
                      ("ms_median", "MEDIAN of the timed launches")):
        print(f"\n=== Speedup over rocSPARSE default -- {what} ===", file=out)
        print(f"{'O':>5}  {'kernel':<22}{'n':>4}{'geomean':>9}{'gstd':>7}{'median':>8}{'min':>7}"
              f"{'max':>8}{'wins':>9}{'max rel_l2':>12}", file=out)
        pooled = {}
        for path in paths:
            with open(path, newline="") as fh:
                first = next(csv.DictReader(fh), None)
            if first is None:
                continue
            O = int(first["O"])
            _, t, _, _ = load(path, col)
            present = {a for m in t for a in t[m]}
            for k in [k for k in kernels if k in present]:
                sp, err = speedups(path, col, k, base)
                if not sp:
                    continue
                pooled.setdefault(k, []).extend(sp)
                s = summary(sp)
                res[(col, O, k)] = dict(s, max_rel_l2=err)
                print(f"{O:>5}  {k:<22}{s['n']:>4}{s['geomean']:>8.2f}x{s['gstd']:>7.2f}"
                      f"{s['median']:>7.2f}x{s['min']:>6.2f}x{s['max']:>7.1f}x"
                      f"{s['wins']:>5}/{s['n']:<3}{err:>12.1e}", file=out)
            print(file=out)
        if len(paths) > 1:
            for k, sp in pooled.items():
                s = summary(sp)
                res[(col, "all", k)] = s
                print(f"{'all':>5}  {k:<22}{s['n']:>4}{s['geomean']:>8.2f}x{s['gstd']:>7.2f}"
                      f"{s['median']:>7.2f}x{s['min']:>6.2f}x{s['max']:>7.1f}x"
                      f"{s['wins']:>5}/{s['n']:<3}", file=out)
    print("\nPer matrix: median over repetitions (fresh processes). "
          "gstd = exp(sigma of log speedup).", file=out)
    return res


# ---- the whole sweep (run.sh) -------------------------------------------------------------
def sweep(corpus, mtxdir, tag="MI355X_S32T128", widths=(128,), tileK=128, segw=32, warmup=3,
          reps=3, algos=None, binary=DRIVER, logdir="logs", outdir="."):
    algos = algos or _env_list("ALGOS", DEFAULT_ALGOS)
    Path(logdir).mkdir(parents=True, exist_ok=True)
    log_path = Path(logdir) / f"run_{tag}.log"
    with open(log_path, "w") as log:
        def say(*a):
            print(*a, file=log, flush=True)
            print(*a, flush=True)
        with open(corpus, newline="") as cf:
            count = sum(1 for _ in csv.DictReader(cf))
        say(f"### host: {socket.gethostname()}   {time.strftime('%Y-%m-%dT%H:%M:%SZ', time.gmtime())}")
        say(f"### corpus: {corpus} ({count} matrices)")
        say(f"### protocol: repeat=10 warmup={warmup}, mean and median recorded; O in "
            f"{{{' '.join(map(str, widths))}}}; tileK=min(O,{tileK}) segw={segw}")
        say(f"### kernels (one process each): {' '.join(algos)}")
        say(f"### repetitions: {reps} per (matrix, kernel); per-matrix median reported")
        csvs = []
        for O in widths:
            tk = min(O, tileK)
            extra = ["--O", str(O), "--tileK", str(tk), "--segw", str(segw), "--repeat", "10",
                     "--warmup", str(warmup), "--stat", "median"]
            path = Path(outdir) / f"results200_{tag}_O{O}.csv"
            say(f"\n### O={O} tileK={tk} -> {path}")
            n = run(binary, corpus, mtxdir, path, algos=algos, reps=reps, extra=extra, log=log)
            say(f"### rows: {n}")
            csvs.append(str(path))
        say("\n### rerunning noisy matrices")
        extra = ["--segw", str(segw), "--repeat", "10", "--warmup", str(warmup), "--stat", "median"]
        rerun_noisy(binary, corpus, mtxdir, csvs, algos=algos, extra=extra, log=log)
        buf = io.StringIO()
        res = table(csvs, out=buf)
        say(buf.getvalue())
    return csvs, res


def main(argv=None):
    p = argparse.ArgumentParser(prog="python -m vcsr_mc_amd.sweep")
    sub = p.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run")
    r.add_argument("binary"), r.add_argument("corpus"), r.add_argument("mtxdir")
    r.add_argument("out")
    q = sub.add_parser("rerun")
    q.add_argument("binary"), q.add_argument("corpus"), q.add_argument("mtxdir")
    q.add_argument("results", nargs="+")
    t = sub.add_parser("table")
    t.add_argument("results", nargs="+")
    a = sub.add_parser("all")
    a.add_argument("--corpus", required=True)
    a.add_argument("--mtx-dir", required=True)
    a.add_argument("--tag", default="MI355X_S32T128")
    a.add_argument("--O", type=int, nargs="+", default=[128])
    a.add_argument("--tileK", type=int, default=128)
    a.add_argument("--segw", type=int, default=32)
    a.add_argument("--warmup", type=int, default=3)
    a.add_argument("--reps", type=int, default=3)
    a.add_argument("--binary", default=str(DRIVER))
    args = p.parse_args(argv)
    if args.cmd == "run":
        run(args.binary, args.corpus, args.mtxdir, args.out)
    elif args.cmd == "rerun":
        rerun_noisy(args.binary, args.corpus, args.mtxdir, args.results)
    elif args.cmd == "table":
        table(args.results)
    else:
        sweep(args.corpus, args.mtx_dir, args.tag, tuple(args.O), args.tileK, args.segw,
              args.warmup, args.reps, binary=args.binary)
    return 0


if __name__ == "__main__":
    sys.exit(main())
