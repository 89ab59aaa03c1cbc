"""The spmm_vcsr driver: the reference's command line, Matrix Market input and CSV output
(src/main.cpp, include/mmio.hpp, include/csr.hpp).  Input errors are raised before any HIP call,
so they are checked without a GPU; the GPU test runs every algorithm with the reference's
two-sided validation."""
import csv
import io
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "vcsr_mc_amd", "spmm_vcsr")


# The reference's CSV schema (src/main.cpp:220), which its analysis scripts read by name.
CSV_HEADER = ("gpu,sm,mtx,O,segw,bundle,tileK,repeat,algo,ms,gflops,validation,rel_l2,setup_ms,"
              "ms_mean,ms_median,convert_ms,upload_ms")


def run(args, timeout=300):
    return subprocess.run([BIN] + args, capture_output=True, text=True, timeout=timeout)


def write_mtx(path, M, N, entries, field="real", sym="general"):
    with open(path, "w") as fh:
        fh.write(f"%%MatrixMarket matrix coordinate {field} {sym}\n% comment\n")
        fh.write(f"{M} {N} {len(entries)}\n")
        for e in entries:
            fh.write(" ".join(str(x) for x in e) + "\n")


@pytest.mark.parametrize("body,msg", [
    ("%%MatrixMarket matrix array real general\n2 2\n1\n2\n3\n4\n", "coordinate"),
    ("%%MatrixMarket matrix coordinate complex general\n2 2 1\n1 1 1 0\n", "Unsupported MTX field"),
    ("%%MatrixMarket matrix coordinate real general\n2 2 2\n1 1 1\n1 1 2\n", "Duplicate"),
    ("%%MatrixMarket matrix coordinate real general\n2 2 1\n3 1 1\n", "out of range"),
    ("%%MatrixMarket matrix coordinate real general\n2 2 2\n1 1 1\n", "Truncated"),
    ("%%MatrixMarket matrix coordinate real symmetric\n2 3 1\n1 1 1\n", "square"),
    ("%%MatrixMarket matrix coordinate real skew-symmetric\n2 2 1\n1 1 5\n", "diagonal"),
])
def test_mtx_errors(tmp_path, body, msg):
    p = tmp_path / "bad.mtx"
    p.write_text(body)
    r = run(["--mtx", str(p), "--O", "8"])
    assert r.returncode == 2 and msg in r.stderr, r.stderr


def test_cli_errors(tmp_path):
    assert run(["--help"]).returncode == 0
    r = run(["--gen", "2:100", "--algo", "nope"])
    assert r.returncode == 2 and "Unknown algorithm" in r.stderr
    r = run(["--gen", "2:100", "--tileK", "48"])
    assert r.returncode == 2 and "tileK" in r.stderr
    r = run(["--gen", "2:100", "--reorder", "amd"])
    assert r.returncode == 2 and "Unknown reordering" in r.stderr


@pytest.mark.gpu
def test_all_algorithms_pass_cpu_check(tmp_path):
    rng = np.random.default_rng(3)
    M = N = 300
    ent = set()
    while len(ent) < 2500:
        r, c = (int(x) for x in rng.integers(1, M + 1, 2))
        if r >= c:
            ent.add((r, c))
    entries = [(r, c, f"{rng.uniform(-1, 1):.6f}") for r, c in sorted(ent)]
    p = tmp_path / "sym.mtx"
    write_mtx(p, M, N, entries, sym="symmetric")
    for segw, tk in ((16, 64), (32, 128)):
        print("[case] driver mtx", segw, tk, flush=True)
        r = run(["--mtx", str(p), "--O", "96", "--segw", str(segw), "--tileK", str(tk),
                 "--check", "cpu", "--csv", "--bdist", "uniform", "--repeat", "3"])
        assert r.returncode == 0, r.stderr
        assert r.stdout.splitlines()[0] == CSV_HEADER
        rows = list(csv.DictReader(io.StringIO(r.stdout)))
        assert {x["algo"] for x in rows} == {"rocsparse", "rocsparse_fp16", "vcsr_mc",
                                             "vcsr_mc_fp32"}
        for x in rows:
            assert x["validation"] == "pass", x
            assert float(x["ms"]) > 0 and float(x["gflops"]) > 0
    print("[case] driver mtx rcm", flush=True)
    r = run(["--mtx", str(p), "--O", "64", "--segw", "32", "--tileK", "64", "--reorder", "rcm",
             "--check", "cpu", "--csv", "--bdist", "normal", "--repeat", "2"])
    assert r.returncode == 0, r.stderr
    rows = list(csv.DictReader(io.StringIO(r.stdout)))
    assert len(rows) == 4 and all(x["validation"] == "pass" for x in rows), rows
    print("[case] driver gen", flush=True)
    r = run(["--gen", "2:3000", "--O", "128", "--segw", "32", "--tileK", "128",
             "--check", "rocsparse", "--csv", "--stat", "median", "--algo", "vcsr_mc,vcsr_mc_fp32"])
    assert r.returncode == 0, r.stderr
    rows = list(csv.DictReader(io.StringIO(r.stdout)))
    assert [x["validation"] for x in rows] == ["pass", "pass"]


def test_dump_csr_matches_reference_reader(tmp_path):
    """The driver's Matrix Market path (include/mmio.hpp + include/csr.hpp) gives, for every
    committed fixture, the CSR the reference's reader builds, or its error text (fixtures written
    by the reference's own headers, tests/golden/make_mtx_golden.py)."""
    import json
    cases = json.load(open(os.path.join(ROOT, "tests", "golden", "mtx_golden.json")))
    for name, case in sorted(cases.items()):
        p = tmp_path / f"{name}.mtx"
        with open(p, "w", newline="") as fh:
            fh.write(case["body"])
        r = run(["--mtx", str(p), "--dump-csr", "-"], timeout=60)
        want = case["reference"]
        if want.startswith("OK"):
            assert r.returncode == 0 and r.stdout == want, (name, r.stderr)
        else:
            assert r.returncode == 2 and r.stderr == f"Error: {want[4:]}", (name, r.stderr)


def test_option_texts():
    """Option errors carry the reference's texts (src/main.cpp:45-53, 136-148, 177)."""
    for args, msg in ((["--O", "0"], "Expected integer >= 1, got: 0"),
                      (["--warmup", "-1"], "Expected integer >= 0, got: -1"),
                      (["--repeat", "12x"], "Expected integer >= 1, got: 12x"),
                      (["--O", "4294967296"], "Expected integer >= 1, got: 4294967296"),
                      (["--check", "gpu"], "Unknown reference: gpu"),
                      (["--stat", "max"], "Unknown --stat: max (mean|median)"),
                      (["--algo", "vcsr_mc,"], "Unknown algorithm: "),
                      (["--bdist", "cauchy"], "Unknown --bdist: cauchy (pattern|normal|uniform|wide)")):
        r = run(["--gen", "1:64"] + args, timeout=60)
        assert r.returncode == 2 and f"Error: {msg}\n" == r.stderr, (args, r.stderr)
    r = run(["--O", "8"], timeout=60)  # no input
    assert r.returncode == 2 and r.stdout.startswith("Usage: spmm_vcsr")
    r = run(["--gen", "1:64", "stray"], timeout=60)
    assert r.returncode == 2 and r.stdout.startswith("Usage: spmm_vcsr")


def _csv_rows(r):
    assert r.returncode == 0, r.stderr
    assert r.stdout.splitlines()[0] == CSV_HEADER
    return {x["algo"]: x for x in csv.DictReader(io.StringIO(r.stdout))}


@pytest.mark.gpu
@pytest.mark.parametrize("bdist", ["pattern", "wide"])
def test_bdist_fills_pass(tmp_path, bdist):
    """The reference's default fill (pattern: 13 values in [-6/7, 6/7], behind all its timings)
    and the wide one (random sign, magnitudes 1e-3..1e3) through every kernel, checked against
    the CPU loop; the default --bdist is pattern."""
    args = ["--gen", "2:2000", "--O", "64", "--segw", "32", "--tileK", "64", "--check", "cpu",
            "--csv", "--repeat", "2"]
    print("[case] driver bdist", bdist, flush=True)
    rows = _csv_rows(run(args + ["--bdist", bdist]))
    assert set(rows) == {"rocsparse", "rocsparse_fp16", "vcsr_mc", "vcsr_mc_fp32"}
    assert all(x["validation"] == "pass" for x in rows.values()), rows
    if bdist == "pattern":
        default = _csv_rows(run(args))
        for k in rows:  # same B, so the same deterministic errors
            assert default[k]["rel_l2"] == rows[k]["rel_l2"] or k.startswith("rocsparse"), k


@pytest.mark.gpu
def test_check_none_and_stat(tmp_path):
    print("[case] driver check none", flush=True)
    rows = _csv_rows(run(["--gen", "1:512", "--O", "32", "--check", "none", "--csv",
                          "--stat", "median", "--algo", "vcsr_mc,vcsr_mc_fp32", "--repeat", "3"]))
    for x in rows.values():
        assert x["validation"] == "unchecked" and float(x["rel_l2"]) == 0
        assert float(x["ms"]) == float(x["ms_median"])


def _cancelling_mtx(path, n=64):
    """Row r: 1.0001 at column r and -1 at column r+1.  With O = 13 every row of the pattern
    fill is the same, so C = 1e-4 x B row: FP16 operands round 1.0001 to 1 and return zeros
    (relative error 1, beyond the FP16 cap of 0.1); FP32 operands meet their bound."""
    entries = [(r + 1, r + 1, "1.0001") for r in range(n)] + \
              [(r + 1, (r + 1) % n + 1, "-1") for r in range(n)]
    write_mtx(path, n, n, entries)


@pytest.mark.gpu
def test_lenient_records_fail(tmp_path):
    p = tmp_path / "cancel.mtx"
    _cancelling_mtx(p)
    base = ["--mtx", str(p), "--O", "13", "--segw", "32", "--tileK", "16", "--check", "cpu",
            "--csv", "--repeat", "2"]
    print("[case] driver lenient fail", flush=True)
    rows = _csv_rows(run(base + ["--lenient"]))
    assert rows["vcsr_mc"]["validation"] == "FAIL" and rows["rocsparse_fp16"]["validation"] == "FAIL"
    assert abs(float(rows["vcsr_mc"]["rel_l2"]) - 1.0) < 1e-6
    assert rows["vcsr_mc_fp32"]["validation"] == "pass" and rows["rocsparse"]["validation"] == "pass"
    r = run(base + ["--algo", "vcsr_mc"])
    assert r.returncode == 2 and "Error: vcsr_mc: correctness check failed, rel_l2=1.000000" in r.stderr


@pytest.mark.gpu
def test_lenient_records_nonfinite(tmp_path):
    """Two values of 3e38 in one row: with O = 13 every row of the pattern fill is
    (k - 6) / 7, so output column 0 is 6e38 x (-6/7), finite in the double CPU loop and an
    overflow in every GPU kernel's FP32 sum.  --lenient records FAIL with rel_l2 = inf; without
    it the driver stops."""
    p = tmp_path / "huge.mtx"
    write_mtx(p, 4, 4, [(1, 1, "3e38"), (1, 2, "3e38"), (2, 2, "1"), (3, 4, "2"), (4, 3, "-1")])
    base = ["--mtx", str(p), "--O", "13", "--segw", "16", "--tileK", "16", "--check", "cpu",
            "--csv", "--repeat", "1", "--warmup", "0", "--bdist", "pattern"]
    print("[case] driver lenient nonfinite", flush=True)
    rows = _csv_rows(run(base + ["--lenient", "--algo", "vcsr_mc,vcsr_mc_fp32,rocsparse"]))
    for k in ("vcsr_mc", "vcsr_mc_fp32", "rocsparse"):
        assert rows[k]["validation"] == "FAIL" and rows[k]["rel_l2"] == "inf", rows[k]
    r = run(base + ["--algo", "vcsr_mc_fp32"])
    assert r.returncode == 2 and "Error: vcsr_mc_fp32: non-finite output" in r.stderr


def test_write_mtx_round_trip(tmp_path):
    """--write-mtx writes the input as a Matrix Market file whose CSR, read back, is the same
    bit for bit (the timing comparison with the reference's driver reads these files)."""
    p = tmp_path / "w.mtx"
    for spec in ("2:3000", "4:40", "5:9"):
        assert run(["--gen", spec, "--write-mtx", str(p)], timeout=120).returncode == 0
        a = run(["--mtx", str(p), "--dump-csr", "-"], timeout=120)
        b = run(["--gen", spec, "--dump-csr", "-"], timeout=120)
        assert a.returncode == 0 and a.stdout == b.stdout, spec
