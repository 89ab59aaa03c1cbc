"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (no GPU): the workload
generators (vcsr_mc_amd/csrc/gen.cpp), the Matrix Market reader and COO -> CSR of the drop-in
headers (include/mmio.hpp, include/csr.hpp, on every committed fixture, error paths included),
and the oracle's C functions.  Each is built with g++/gcc -fsanitize=address,undefined and
-fno-sanitize-recover, so any report fails the run."""
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HERE = os.path.join(ROOT, "tests", "sanitize")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
       "-g", "-O1"]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
           UBSAN_OPTIONS="print_stacktrace=1", OMP_NUM_THREADS="4")


def build(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]


def run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True, env=ENV, timeout=600)
    assert r.returncode == 0 and "runtime error" not in r.stderr and "ERROR:" not in r.stderr, \
        (r.stdout[-1000:], r.stderr[-3000:])
    return r.stdout


def test_generators(tmp_path):
    exe = str(tmp_path / "gen")
    build(["g++", "-std=c++17", "-fopenmp", *SAN, f"-I{ROOT}/include",
           os.path.join(ROOT, "vcsr_mc_amd", "csrc", "gen.cpp"),
           os.path.join(HERE, "gen_harness.cpp"), "-o", exe])
    assert run([exe]).endswith("ok\n")


def test_mtx_reader(tmp_path):
    exe = str(tmp_path / "mtx")
    build(["g++", "-std=c++17", *SAN, f"-I{ROOT}/include", os.path.join(ROOT, "oracle",
                                                                        "mtx_dump.cpp"),
           "-o", exe])
    cases = json.load(open(os.path.join(ROOT, "tests", "golden", "mtx_golden.json")))
    for name, case in cases.items():
        p = tmp_path / f"{name}.mtx"
        with open(p, "w", newline="") as fh:
            fh.write(case["body"])
        assert run([exe, str(p)]) == case["reference"], name


def test_oracle(tmp_path):
    exe = str(tmp_path / "orc")
    build(["gcc", "-std=c99", "-fopenmp", *SAN, f"-I{ROOT}/oracle",
           os.path.join(ROOT, "oracle", "vcsrmc_oracle.c"),
           os.path.join(ROOT, "oracle", "rcm_oracle.c"), os.path.join(HERE, "oracle_harness.c"),
           "-lm", "-o", exe])
    assert run([exe]).endswith("ok\n")
