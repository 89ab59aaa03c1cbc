"""The corpus sweep protocol (vcsr_mc_amd/sweep.py; the reference's bench200/run200.py,
rerun_noisy.py, analyze.py, orig_table.py): statistics against closed forms, and the run /
rerun / report logic against a stub driver whose timings are known, so no GPU is needed.  The
GPU test runs the real spmm_vcsr over a small corpus."""
import csv
import io
import math
import os
import stat
import sys

import numpy as np
import pytest

from vcsr_mc_amd import sweep

STUB = r'''#!/usr/bin/env python3
# Stand-in for spmm_vcsr: one CSV row per call.  ms = base[matrix] * factor[algo]; a matrix
# named noisy* is 10x slower on the first call of each algorithm (a slow process); algo "bad"
# fails.  Calls are counted in a state file next to this script.
import json, os, sys
args = sys.argv[1:]
opt = {args[i]: args[i + 1] for i in range(0, len(args) - 1) if args[i].startswith("--")}
mtx, algo = opt["--mtx"], opt["--algo"]
name = os.path.basename(mtx)[:-4]
if algo == "bad":
    sys.stderr.write("Unknown algorithm: bad\n"); sys.exit(2)
state = os.path.join(os.path.dirname(os.path.abspath(__file__)), "calls.json")
calls = json.load(open(state)) if os.path.exists(state) else {}
key = name + "/" + algo
calls[key] = calls.get(key, 0) + 1
json.dump(calls, open(state, "w"))
base = {"a": 1.0, "b": 2.0, "noisy": 4.0}[name]
factor = {"rocsparse": 1.0, "rocsparse_fp16": 1.2, "vcsr_mc": 0.25, "vcsr_mc_fp32": 0.5}[algo]
ms = base * factor * (10.0 if name == "noisy" and calls[key] == 1 else 1.0)
mflop = 100.0 * base
O = opt.get("--O", "128"); tk = opt.get("--tileK", "64")
print("gpu,sm,mtx,O,segw,bundle,tileK,repeat,algo,ms,gflops,validation,rel_l2,setup_ms,"
      "ms_mean,ms_median,convert_ms,upload_ms")
print(f"stub,gfx950,{mtx},{O},32,16,{tk},10,{algo},{ms},{mflop / ms},pass,{1e-7 * factor},0,"
      f"{ms * 1.1},{ms},0.5,0.25")
'''


@pytest.fixture
def stub(tmp_path):
    p = tmp_path / "bin" / "spmm_stub"
    p.parent.mkdir()
    p.write_text(STUB.replace("/usr/bin/env python3", sys.executable, 1))
    p.chmod(p.stat().st_mode | stat.S_IEXEC)
    return p


@pytest.fixture
def corpus(tmp_path):
    d = tmp_path / "mtx"
    d.mkdir()
    for n in ("a", "b", "noisy"):
        (d / f"{n}.mtx").write_text("%%MatrixMarket matrix coordinate real general\n1 1 1\n1 1 1\n")
    c = tmp_path / "corpus.csv"
    c.write_text("group,name,rows,cols,nnz\ng,a,1,1,10\ng,b,1,1,20\ng,noisy,1,1,30\n"
                 "g,absent,1,1,40\n")
    return c, d


def rows_of(path):
    with open(path, newline="") as fh:
        return list(csv.DictReader(fh))


# The reference sweep's results columns (bench200/run200.py:22-24), read by name by its
# rerun and table scripts.
RESULT_FIELDS = ["gpu", "sm", "mtx", "O", "segw", "bundle", "tileK", "repeat", "algo", "ms",
                 "gflops", "validation", "rel_l2", "setup_ms", "nnz", "rep", "ms_mean",
                 "ms_median", "convert_ms", "upload_ms"]


def test_result_columns_match_reference():
    assert sweep.RESULT_COLUMNS == RESULT_FIELDS


def test_synth_corpus_files(tmp_path):
    """The synthetic corpus at a tiny scale: 24 valid Matrix Market files whose header counts,
    entries and corpus row agree (distinct, in range, row-major)."""
    from vcsr_mc_amd import synth_corpus
    path = synth_corpus.make(str(tmp_path), scale=0.002)
    rows = rows_of(path)
    assert len(rows) == 24 and len({r["name"] for r in rows}) == 24
    for r in rows:
        lines = (tmp_path / "mtx" / f"{r['name']}.mtx").read_text().splitlines()
        assert lines[0] == "%%MatrixMarket matrix coordinate real general"
        M, N, nnz = (int(x) for x in lines[1].split())
        assert (M, N, nnz) == (int(r["rows"]), int(r["cols"]), int(r["nnz"])) and nnz > 0
        e = np.array([[int(a), int(b)] for a, b, _ in (x.split() for x in lines[2:])])
        assert len(e) == nnz
        assert e[:, 0].min() >= 1 and e[:, 0].max() <= M and e[:, 1].min() >= 1
        assert e[:, 1].max() <= N
        key = (e[:, 0] - 1) * N + (e[:, 1] - 1)
        assert np.all(np.diff(key) > 0)


def test_statistics_closed_forms():
    assert sweep.median([3, 1, 2]) == 2 and sweep.median([4, 1, 3, 2]) == 2.5
    gm, gs = sweep.geo_gstd([2.0, 8.0])  # logs ln2, ln8: mean ln4, sigma ln2
    assert math.isclose(gm, 4.0) and math.isclose(gs, 2.0)
    gm, gs = sweep.geo_gstd([5.0] * 7)
    assert math.isclose(gm, 5.0) and math.isclose(gs, 1.0)
    assert all(math.isnan(x) for x in sweep.geo_gstd([]))
    assert sweep.matrix_of("/x/y/cop20k_A.mtx") == "cop20k_A"
    assert sweep.with_width(["--repeat", "10", "--O", "7", "--tileK", "16"], 128, 64) == \
        ["--O", "128", "--tileK", "64", "--repeat", "10"]


def test_run_writes_reference_columns(stub, corpus, tmp_path):
    c, d = corpus
    out = tmp_path / "r.csv"
    log = io.StringIO()
    n = sweep.run(stub, c, d, out, algos=["rocsparse", "vcsr_mc", "bad"], reps=2,
                  extra=["--O", "64", "--tileK", "64"], log=log)
    rows = rows_of(out)
    assert n == len(rows) == 3 * 2 * 2  # 3 present matrices x 2 reps x 2 working algos
    assert list(rows[0].keys()) == sweep.RESULT_COLUMNS
    assert {r["rep"] for r in rows} == {"0", "1"}
    assert {r["nnz"] for r in rows if sweep.matrix_of(r["mtx"]) == "b"} == {"20"}
    assert all(r["O"] == "64" for r in rows)
    text = log.getvalue()
    assert "absent: no Matrix Market file at" in text and "absent.mtx, skipped" in text
    assert "a / bad / repetition 0: Unknown algorithm: bad" in text
    assert "b: 4 rows" in text  # 2 repetitions x 2 working kernels


def test_load_medians_and_gflops(stub, corpus, tmp_path):
    c, d = corpus
    out = tmp_path / "r.csv"
    sweep.run(stub, c, d, out, algos=["rocsparse", "vcsr_mc"], reps=3, log=io.StringIO())
    res = sweep.Results.read(out, "ms")
    assert res.time("a", "vcsr_mc") == 0.25 and res.time("b", "rocsparse") == 2.0
    # noisy: first call 10x slower, median of three is the normal time
    assert res.time("noisy", "vcsr_mc") == 1.0
    assert math.isclose(res.gflops("b", "vcsr_mc"), 200.0 / 0.5)
    mean = sweep.Results.read(out, "ms_mean")
    assert math.isclose(mean.time("a", "rocsparse"), 1.1)
    assert math.isclose(mean.gflops("a", "rocsparse"), 100.0 / 1.1)
    assert math.isclose(res.error("a", "vcsr_mc"), 0.25e-7) and res.nnz["noisy"] == 30
    assert res.width == 128
    assert res.speedups("vcsr_mc") == {"a": 4.0, "b": 4.0, "noisy": 4.0}


def test_rerun_replaces_noisy_rows(stub, corpus, tmp_path):
    c, d = corpus
    out = tmp_path / "results_O128.csv"
    sweep.run(stub, c, d, out, algos=["rocsparse", "vcsr_mc"], reps=2, log=io.StringIO())
    before = rows_of(out)
    assert sweep.noisy_matrices(before) == ["noisy"]
    done = sweep.rerun_noisy(stub, c, d, [out], algos=["rocsparse", "vcsr_mc"],
                             extra=["--O", "999", "--repeat", "10"], log=io.StringIO())
    assert done[str(out)] == ["noisy"]
    after = rows_of(out)
    raw = rows_of(tmp_path / "results_O128_raw.csv")
    assert raw == before
    noisy_rows = [r for r in after if sweep.matrix_of(r["mtx"]) == "noisy"]
    assert len(noisy_rows) == sweep.NOISY_REPS * 2
    assert all(float(r["ms"]) < 10 for r in noisy_rows)  # later calls are not slow
    assert all(r["O"] == "128" for r in noisy_rows)  # --O comes from the results file
    assert [r for r in after if sweep.matrix_of(r["mtx"]) != "noisy"] == \
        [r for r in before if sweep.matrix_of(r["mtx"]) != "noisy"]
    assert not (tmp_path / "results_O128_rerun_corpus.csv").exists()


def test_report_speedups(stub, corpus, tmp_path):
    c, d = corpus
    paths = []
    for O in (64, 128):
        p = tmp_path / f"res_O{O}.csv"
        sweep.run(stub, c, d, p, algos=sweep.ALL_KERNELS, reps=3,
                  extra=["--O", str(O)], log=io.StringIO())
        paths.append(str(p))
    buf = io.StringIO()
    res = sweep.report(paths, out=buf)
    s = res[("ms_median", 64, "vcsr_mc")]
    assert s.n == 3 and math.isclose(s.geomean, 4.0) and math.isclose(s.gstd, 1.0)
    assert s.wins == 3 and math.isclose(s.max_rel_l2, 0.25e-7)
    assert s.min == s.max == s.median == 4.0
    assert math.isclose(res[("ms_median", "all", "vcsr_mc_fp32")].geomean, 2.0)
    assert res[("ms_median", "all", "vcsr_mc_fp32")].n == 6
    assert math.isclose(res[("ms_mean", 128, "vcsr_mc")].geomean, 4.0)
    text = buf.getvalue()
    assert "Speedup over rocsparse" in text and "| 64 | vcsr_mc | 3 | 4.00x |" in text


@pytest.mark.gpu
def test_sweep_real_driver(tmp_path):
    """The whole protocol with the real driver over three small Matrix Market files."""
    rng = np.random.default_rng(8)
    d = tmp_path / "mtx"
    d.mkdir()
    lines = ["group,name,rows,cols,nnz"]
    for i, n in enumerate((200, 350, 500)):
        ent = set()
        while len(ent) < 6 * n:
            ent.add((int(rng.integers(1, n + 1)), int(rng.integers(1, n + 1))))
        with open(d / f"m{i}.mtx", "w") as fh:
            fh.write(f"%%MatrixMarket matrix coordinate real general\n{n} {n} {len(ent)}\n")
            for r, cc in sorted(ent):
                fh.write(f"{r} {cc} {rng.uniform(-1, 1):.6f}\n")
        lines.append(f"g,m{i},{n},{n},{len(ent)}")
    c = tmp_path / "corpus.csv"
    c.write_text("\n".join(lines) + "\n")
    print("[case] sweep over 3 matrices", flush=True)
    csvs, res = sweep.sweep(c, d, tag="t", widths=(32,), tileK=128, reps=2,
                            logdir=tmp_path / "logs", outdir=tmp_path)
    rows = rows_of(csvs[0])
    assert len(rows) == 3 * 2 * len(sweep.ALL_KERNELS)
    assert all(r["validation"] == "pass" for r in rows)
    assert all(r["tileK"] == "32" for r in rows)
    for k in sweep.REPORTED:
        assert res[("ms_median", 32, k)].n == 3
