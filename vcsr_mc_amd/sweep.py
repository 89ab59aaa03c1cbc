"""Corpus sweep for the spmm_vcsr driver: measure, re-measure noisy matrices, report speedups.

The protocol of the reference's corpus harness (bench200/run200.py, rerun_noisy.py, analyze.py,
orig_table.py, run.sh of MuuSeoTia/VCSR_MC), over Matrix Market files supplied locally (nothing
is downloaded).  What is kept from it is the interface: the results CSV columns and file names,
the environment variables ALGOS / REPS / EXTRA, the noise rule and the statistics.  The code is
organised differently:

* a sweep is a plan of jobs (matrix, repetition, kernel), each run by a `Driver` -- one fresh
  process of the binary with ``--mtx --algo --csv`` and the sweep's extra arguments -- whose rows
  are tagged with the corpus nnz and the repetition and streamed to the CSV;
* `Results` holds a CSV's rows per (matrix, kernel) cell: the median time over repetitions, the
  GFLOP/s at that time (from the FLOP count every row of a matrix shares) and the largest
  rel_l2;
* a matrix is noisy when some kernel's slowest repetition took more than twice its fastest;
  `rerun_noisy` measures those matrices again with five fresh repetitions, in memory, and
  replaces their rows, keeping the first CSV as ``<name>_raw.csv``;
* `report` prints, per timing column (mean and median of a process's timed launches) and width
  O, each kernel's speedup over rocSPARSE (t_rocsparse / t_kernel per matrix) as geometric mean,
  geometric standard deviation exp(sigma of ln speedup), median, min, max, wins and the largest
  rel_l2, pooled over widths when several CSVs are given.

Usage::

    python -m vcsr_mc_amd.sweep run    BINARY CORPUS.csv MTXDIR OUT.csv
    python -m vcsr_mc_amd.sweep rerun  BINARY CORPUS.csv MTXDIR RESULTS.csv [...]
    python -m vcsr_mc_amd.sweep report RESULTS.csv [...]
    python -m vcsr_mc_amd.sweep all    --corpus CORPUS.csv --mtx-dir MTXDIR [--tag T] [--O 128 ...]
"""
from __future__ import annotations

import argparse
import csv
import io
import math
import os
import platform
import shlex
import shutil
import statistics
import subprocess
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable, Iterable

# Columns of a results CSV (the reference harness's, bench200/run200.py:22-24): the driver's CSV
# columns plus the corpus nnz and the repetition.
RESULT_COLUMNS = ["gpu", "sm", "mtx", "O", "segw", "bundle", "tileK", "repeat", "algo", "ms",
                  "gflops", "validation", "rel_l2", "setup_ms", "nnz", "rep", "ms_mean",
                  "ms_median", "convert_ms", "upload_ms"]
ALL_KERNELS = ("rocsparse", "rocsparse_fp16", "vcsr_mc", "vcsr_mc_fp32")
BASELINE = "rocsparse"
REPORTED = ("vcsr_mc", "vcsr_mc_fp32")
NOISE_SPREAD = 2.0   # slowest / fastest repetition above this: the matrix is measured again
NOISY_REPS = 5       # repetitions of a noisy matrix's second measurement
RERUN_KERNELS = ("rocsparse", "vcsr_mc")
RERUN_EXTRA = "--repeat 10 --warmup 0 --stat median"
DRIVER = Path(__file__).resolve().parent / "spmm_vcsr"


def _from_env(name: str, fallback: Iterable[str]) -> list[str]:
    """A list option from the environment (spaces or commas), else the fallback."""
    text = os.environ.get(name, "")
    return text.replace(",", " ").split() if text.strip() else list(fallback)


def matrix_of(mtx_path: str) -> str:
    """Corpus name of a row's Matrix Market path: its file name without .mtx."""
    stem = Path(mtx_path.replace("\\", "/")).name
    return stem[: -len(".mtx")] if stem.endswith(".mtx") else stem


# ---- statistics -------------------------------------------------------------------------------
def median(values: Iterable[float]) -> float:
    return statistics.median(list(values))


def geo_gstd(values: Iterable[float]) -> tuple[float, float]:
    """Geometric mean and geometric standard deviation, exp(population sigma of ln x)."""
    logs = [math.log(v) for v in values]
    if not logs:
        return math.nan, math.nan
    return math.exp(statistics.fmean(logs)), math.exp(statistics.pstdev(logs))


# ---- running the driver -----------------------------------------------------------------------
@dataclass(frozen=True)
class Job:
    matrix: str
    path: Path
    nnz: str
    algo: str
    rep: int


@dataclass
class Outcome:
    job: Job
    rows: list = field(default_factory=list)
    problem: str | None = None  # why the job gave no rows


class Driver:
    """Runs one job as a fresh process of the benchmark binary."""

    def __init__(self, binary, extra: Iterable[str] = (), timeout: float = 300):
        self.binary = str(binary)
        self.extra = list(extra)
        self.timeout = timeout

    def __call__(self, job: Job) -> Outcome:
        argv = [self.binary, "--mtx", str(job.path), "--algo", job.algo, "--csv", *self.extra]
        try:
            proc = subprocess.run(argv, capture_output=True, text=True, timeout=self.timeout)
        except subprocess.TimeoutExpired:
            return Outcome(job, problem=f"no result within {self.timeout:g} s")
        if proc.returncode != 0:
            lines = [l for l in (proc.stderr or "").splitlines() if l.strip()]
            return Outcome(job, problem=lines[-1].strip() if lines
                           else f"exit status {proc.returncode}")
        rows = []
        for row in csv.DictReader(io.StringIO(proc.stdout)):
            row.update(nnz=job.nnz, rep=job.rep)
            rows.append(row)
        return Outcome(job, rows)


def read_corpus(path) -> list[dict]:
    with open(path, newline="") as fh:
        return list(csv.DictReader(fh))


def plan(entries: Iterable[dict], mtxdir, algos: Iterable[str], reps: int,
         say: Callable[[str], None]) -> list[Job]:
    """Jobs for the corpus entries whose file exists: per matrix, every repetition runs every
    kernel once (so a slow process hits one repetition of all kernels, not one kernel)."""
    jobs = []
    for entry in entries:
        path = Path(mtxdir) / f"{entry['name']}.mtx"
        if not path.is_file():
            say(f"{entry['name']}: no Matrix Market file at {path}, skipped")
            continue
        jobs += [Job(entry["name"], path, entry.get("nnz", ""), algo, rep)
                 for rep in range(reps) for algo in algos]
    return jobs


def execute(jobs: list[Job], driver: Callable[[Job], Outcome], emit: Callable[[list], None],
            say: Callable[[str], None]) -> int:
    """Runs the jobs in order, passing each job's rows to `emit`; returns the rows emitted."""
    count, done = 0, None
    for job in jobs:
        if done is not None and job.matrix != done[0]:
            say(f"{done[0]}: {done[1]} rows")
            done = None
        out = driver(job)
        if out.problem is not None:
            say(f"{job.matrix} / {job.algo} / repetition {job.rep}: {out.problem}")
        else:
            emit(out.rows)
            count += len(out.rows)
        done = (job.matrix, (done[1] if done else 0) + len(out.rows))
    if done is not None:
        say(f"{done[0]}: {done[1]} rows")
    return count


def _logger(stream):
    def say(text):
        print(text, file=stream, flush=True)
    return say


def run(binary, corpus, mtxdir, out, algos=None, reps=None, extra=None, timeout=300,
        log=None) -> int:
    """Measures every (matrix, repetition, kernel) of the corpus into the CSV `out`; returns the
    number of rows written.  Unset options come from ALGOS, REPS and EXTRA."""
    algos = list(algos) if algos else _from_env("ALGOS", ALL_KERNELS)
    reps = int(os.environ.get("REPS", "1")) if reps is None else reps
    extra = shlex.split(os.environ.get("EXTRA", "")) if extra is None else list(extra)
    say = _logger(log or sys.stderr)
    jobs = plan(read_corpus(corpus), mtxdir, algos, reps, say)
    with open(out, "w", newline="") as fh:
        sink = csv.DictWriter(fh, fieldnames=RESULT_COLUMNS, extrasaction="ignore")
        sink.writeheader()

        def emit(rows):
            sink.writerows(rows)
            fh.flush()

        return execute(jobs, Driver(binary, extra, timeout), emit, say)


# ---- results ----------------------------------------------------------------------------------
@dataclass
class Cell:
    """One (matrix, kernel) of a results CSV: its repetitions."""
    times: list = field(default_factory=list)
    errors: list = field(default_factory=list)

    @property
    def time(self) -> float:
        return median(self.times)

    @property
    def max_error(self) -> float:
        return max(self.errors)


class Results:
    """A results CSV per (matrix, kernel), timed by one of its timing columns."""

    def __init__(self, rows: Iterable[dict], column: str = "ms"):
        self.column = column
        self.cells: dict[tuple[str, str], Cell] = {}
        self.mflop: dict[str, float] = {}  # FLOP count / 1e6, shared by a matrix's rows
        self.nnz: dict[str, int] = {}
        self.width = None
        for row in rows:
            m = matrix_of(row["mtx"])
            cell = self.cells.setdefault((m, row["algo"]), Cell())
            cell.times.append(float(row[column]))
            cell.errors.append(float(row["rel_l2"]))
            if float(row["ms"]) > 0:
                self.mflop[m] = float(row["gflops"]) * float(row["ms"])
            self.nnz[m] = int(row["nnz"]) if row.get("nnz") else 0
            if self.width is None:
                self.width = int(row["O"])

    @classmethod
    def read(cls, path, column: str = "ms") -> "Results":
        with open(path, newline="") as fh:
            return cls(csv.DictReader(fh), column)

    def time(self, matrix: str, algo: str) -> float:
        return self.cells[(matrix, algo)].time

    def gflops(self, matrix: str, algo: str) -> float:
        t = self.time(matrix, algo)
        return self.mflop.get(matrix, 0.0) / t if t > 0 else 0.0

    def error(self, matrix: str, algo: str) -> float:
        return self.cells[(matrix, algo)].max_error

    def algos(self) -> set:
        return {a for _, a in self.cells}

    def speedups(self, kernel: str, base: str = BASELINE) -> dict[str, float]:
        """t_base / t_kernel for every matrix timed (above zero) for both."""
        out = {}
        for (m, a), cell in self.cells.items():
            if a != kernel or (m, base) not in self.cells:
                continue
            tk, tb = cell.time, self.time(m, base)
            if tk > 0 and tb > 0:
                out[m] = tb / tk
        return out


# ---- noisy matrices ---------------------------------------------------------------------------
def noisy_matrices(rows: Iterable[dict], spread: float = NOISE_SPREAD) -> list[str]:
    """Matrices where some kernel's slowest repetition took more than `spread` x its fastest."""
    lo: dict = {}
    hi: dict = {}
    for row in rows:
        key, t = (matrix_of(row["mtx"]), row["algo"]), float(row["ms"])
        lo[key] = min(lo.get(key, t), t)
        hi[key] = max(hi.get(key, t), t)
    return sorted({m for (m, a) in lo if lo[(m, a)] > 0 and hi[(m, a)] > spread * lo[(m, a)]})


def with_width(extra: Iterable[str], O, tileK) -> list[str]:
    """`extra` with its --O / --tileK pairs replaced by the given ones."""
    kept, tokens = [], iter(extra)
    for tok in tokens:
        if tok in ("--O", "--tileK"):
            next(tokens, None)
        else:
            kept.append(tok)
    return ["--O", str(O), "--tileK", str(tileK), *kept]


def rerun_noisy(binary, corpus, mtxdir, paths, algos=None, extra=None, reps=NOISY_REPS,
                spread=NOISE_SPREAD, log=None) -> dict:
    """Measures each results CSV's noisy matrices again (`reps` fresh repetitions, the CSV's own
    O and tileK) and replaces their rows in place; the first version of each CSV stays as
    <name>_raw.csv.  Returns {path: noisy matrices}."""
    algos = list(algos) if algos else _from_env("ALGOS", RERUN_KERNELS)
    extra = shlex.split(os.environ.get("EXTRA", RERUN_EXTRA)) if extra is None else list(extra)
    say = _logger(log or sys.stdout)
    entries = read_corpus(corpus)
    found = {}
    for path in map(Path, paths):
        raw = path.with_name(f"{path.stem}_raw.csv")
        if not raw.exists():
            shutil.copy(path, raw)
        with raw.open(newline="") as fh:
            first = list(csv.DictReader(fh))
        noisy = noisy_matrices(first, spread)
        found[str(path)] = noisy
        if not first:
            continue
        say(f"{path.name} (O = {first[0]['O']}): {len(noisy)} noisy matrices"
            + (f" -- {', '.join(noisy)}" if noisy else ""))
        if not noisy:
            continue
        driver = Driver(binary, with_width(extra, first[0]["O"], first[0]["tileK"]))
        fresh: list = []
        jobs = plan([e for e in entries if e["name"] in noisy], mtxdir, algos, reps, say)
        execute(jobs, driver, fresh.extend, lambda _text: None)
        with path.open("w", newline="") as fh:
            w = csv.DictWriter(fh, fieldnames=list(first[0]), extrasaction="ignore")
            w.writeheader()
            w.writerows(r for r in first if matrix_of(r["mtx"]) not in noisy)
            w.writerows(fresh)
        say(f"  {len(fresh)} rows from {reps} new repetitions now stand for them in {path.name}")
    return found


# ---- report -----------------------------------------------------------------------------------
@dataclass
class Summary:
    n: int
    geomean: float
    gstd: float
    median: float
    min: float
    max: float
    wins: int
    max_rel_l2: float = math.nan


def summarize(speedups: list[float], max_rel_l2: float = math.nan) -> Summary:
    gm, gs = geo_gstd(speedups)
    return Summary(len(speedups), gm, gs, median(speedups), min(speedups), max(speedups),
                   sum(1 for s in speedups if s > 1.0), max_rel_l2)


def _line(width, kernel: str, s: Summary) -> str:
    err = "" if math.isnan(s.max_rel_l2) else f"{s.max_rel_l2:.1e}"
    return (f"| {width} | {kernel} | {s.n} | {s.geomean:.2f}x | {s.gstd:.2f} | {s.median:.2f}x "
            f"| {s.min:.2f}x | {s.max:.1f}x | {s.wins}/{s.n} | {err} |")


def report(paths, kernels=REPORTED, base=BASELINE, out=None) -> dict:
    """Prints the speedup tables (Markdown) and returns {(column, O or 'all', kernel): Summary}."""
    out = out or sys.stdout
    found = {}
    for column, what in (("ms_mean", "mean"), ("ms_median", "median")):
        print(f"\n### Speedup over {base} (its default algorithm), by the {what} of each "
              f"process's timed launches\n", file=out)
        print("| O | kernel | matrices | geomean | gstd | median | min | max | wins | "
              "max rel_l2 |", file=out)
        print("|---|---|---|---|---|---|---|---|---|---|", file=out)
        pooled: dict[str, list] = {}
        for path in paths:
            res = Results.read(path, column)
            if res.width is None:
                continue
            for k in (k for k in kernels if k in res.algos()):
                sp = res.speedups(k, base)
                if not sp:
                    continue
                err = max(res.error(m, a) for (m, a) in res.cells if a == k)
                s = summarize(list(sp.values()), err)
                found[(column, res.width, k)] = s
                pooled.setdefault(k, []).extend(sp.values())
                print(_line(res.width, k, s), file=out)
        if len(paths) > 1:
            for k, sp in pooled.items():
                s = summarize(sp)
                found[(column, "all", k)] = s
                print(_line("all", k, s), file=out)
    print("\nEach matrix counts once per width: the median of its repetitions, each a fresh "
          "process. gstd = exp(standard deviation of ln speedup).", file=out)
    return found


# ---- the whole sweep --------------------------------------------------------------------------
def sweep(corpus, mtxdir, tag="MI355X_S32T128", widths=(128,), tileK=128, segw=32, warmup=3,
          reps=3, algos=None, binary=DRIVER, logdir="logs", outdir="."):
    """Every width O: measure the corpus into results200_<tag>_O<O>.csv; then re-measure noisy
    matrices and report.  Returns (CSV paths, report summaries)."""
    algos = list(algos) if algos else _from_env("ALGOS", ALL_KERNELS)
    Path(logdir).mkdir(parents=True, exist_ok=True)
    with open(Path(logdir) / f"run_{tag}.log", "w") as logf:
        def say(text):
            print(text, file=logf, flush=True)
            print(text, flush=True)

        entries = read_corpus(corpus)
        say(f"sweep {tag} on {platform.node()} at "
            f"{time.strftime('%Y-%m-%d %H:%M:%S UTC', time.gmtime())}")
        say(f"  corpus {corpus}: {len(entries)} matrices; kernels {', '.join(algos)}, "
            f"each in its own process, {reps} repetitions (median kept)")
        say(f"  widths O = {', '.join(map(str, widths))}; tileK = min(O, {tileK}); segw {segw}; "
            f"10 timed launches after {warmup} warm-ups, mean and median")
        paths = []
        for O in widths:
            tk = min(O, tileK)
            common = ["--segw", str(segw), "--repeat", "10", "--warmup", str(warmup), "--stat",
                      "median"]
            path = Path(outdir) / f"results200_{tag}_O{O}.csv"
            n = run(binary, corpus, mtxdir, path, algos=algos, reps=reps,
                    extra=with_width(common, O, tk), log=logf)
            say(f"  O = {O}: {n} rows in {path}")
            paths.append(str(path))
        rerun_noisy(binary, corpus, mtxdir, paths, algos=algos,
                    extra=["--segw", str(segw), "--repeat", "10", "--warmup", str(warmup),
                           "--stat", "median"], log=logf)
        text = io.StringIO()
        found = report(paths, out=text)
        say(text.getvalue())
    return paths, found


def main(argv=None) -> int:
    p = argparse.ArgumentParser(prog="python -m vcsr_mc_amd.sweep")
    sub = p.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run", help="measure a corpus into one results CSV")
    for name in ("binary", "corpus", "mtxdir", "out"):
        r.add_argument(name)
    q = sub.add_parser("rerun", help="re-measure the noisy matrices of results CSVs")
    for name in ("binary", "corpus", "mtxdir"):
        q.add_argument(name)
    q.add_argument("results", nargs="+")
    t = sub.add_parser("report", help="speedup tables of results CSVs")
    t.add_argument("results", nargs="+")
    a = sub.add_parser("all", help="measure every width, re-measure noisy matrices, report")
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
    elif args.cmd == "report":
        report(args.results)
    else:
        sweep(args.corpus, args.mtx_dir, args.tag, tuple(args.O), args.tileK, args.segw,
              args.warmup, args.reps, binary=args.binary)
    return 0


if __name__ == "__main__":
    sys.exit(main())
