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
