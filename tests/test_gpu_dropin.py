"""The reference's own driver (src/main.cpp + src/kernels.cu, compiled from its sources against
this repository's include/ and linked with libvcsrmc.so: oracle/_ref/spmm_vcsr_dropin) runs this
library's VCSR-MC path on the GPU and passes its own validation (main.cpp:257-291) against its
CPU loop and against hipSPARSE, with and without --reorder rcm.  The binary is built in the
build container, where the reference sources are, and travels with the tree; without it these
tests skip."""
import os
import subprocess

import numpy as np
import pytest

import vcsr_mc_amd as vm
from gpu_util import say

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DROPIN = os.path.join(ROOT, "oracle", "_ref", "spmm_vcsr_dropin")


def write_mtx(path, A, symmetric=False):
    rows = np.repeat(np.arange(A.M), np.diff(A.row_ptr)) + 1
    with open(path, "w") as fh:
        kind = "symmetric" if symmetric else "general"
        keep = rows >= A.col + 1 if symmetric else np.ones(A.nnz, bool)
        fh.write(f"%%MatrixMarket matrix coordinate real {kind}\n")
        fh.write(f"{A.M} {A.N} {int(keep.sum())}\n")
        for r, c, v in zip(rows[keep], A.col[keep] + 1, A.val[keep]):
            fh.write(f"{r} {c} {float(v)!r}\n")


@pytest.fixture(scope="module")
def mtx(tmp_path_factory):
    if not os.path.exists(DROPIN):
        pytest.skip("oracle/_ref/spmm_vcsr_dropin not built (needs the reference sources)")
    d = tmp_path_factory.mktemp("dropin")
    path = str(d / "powerlaw3000.mtx")
    write_mtx(path, vm.generate(2, 3000), symmetric=True)
    return path


def run(args):
    say("reference driver", *args)
    r = subprocess.run([DROPIN, *args], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-2000:]
    rows = [l.split(",") for l in r.stdout.splitlines()[1:] if l.strip()]
    return {row[8]: row for row in rows}


@pytest.mark.parametrize("check", ["cpu", "rocsparse"])
@pytest.mark.parametrize("reorder", ["none", "rcm"])
def test_reference_driver_validates_library(mtx, check, reorder):
    rows = run(["--mtx", mtx, "--O", "128", "--segw", "32", "--tileK", "128", "--repeat", "3",
                "--warmup", "1", "--algo", "vcsr_mc,vcsr_mc_fp32,rocsparse", "--check", check,
                "--reorder", reorder, "--bdist", "uniform", "--csv"])
    assert set(rows) == {"vcsr_mc", "vcsr_mc_fp32", "rocsparse"}
    for name in ("vcsr_mc", "vcsr_mc_fp32"):
        assert rows[name][11] == "pass", rows[name]
        rel = float(rows[name][12])
        assert rel < (2e-3 if name == "vcsr_mc" else 1e-5), rows[name]


@pytest.mark.parametrize("segw,tileK,O", [(16, 64, 128), (48, 32, 100), (64, 16, 7)])
def test_reference_driver_other_shapes(mtx, segw, tileK, O):
    rows = run(["--mtx", mtx, "--O", str(O), "--segw", str(segw), "--tileK", str(tileK),
                "--repeat", "2", "--warmup", "1", "--algo", "vcsr_mc,vcsr_mc_fp32",
                "--check", "cpu", "--csv"])
    for name in ("vcsr_mc", "vcsr_mc_fp32"):
        assert rows[name][11] == "pass", rows[name]


DRIVER = os.path.join(ROOT, "vcsr_mc_amd", "spmm_vcsr")


@pytest.mark.parametrize("config,O,check", [(1, 128, "cpu"), (2, 128, "cpu"),
                                            (3, 128, "rocsparse"), (4, 256, "rocsparse")])
def test_reference_driver_full_workloads(tmp_path, config, O, check):
    """The reference's driver validates both of this library's kernels on full benchmark
    workloads: the Matrix Market file spmm_vcsr --gen K --write-mtx writes, read by the
    reference's own reader, checked against its CPU loop or hipSPARSE."""
    if not os.path.exists(DROPIN):
        pytest.skip("oracle/_ref/spmm_vcsr_dropin not built (needs the reference sources)")
    path = str(tmp_path / f"workload{config}.mtx")
    say("write workload", config)
    subprocess.run([DRIVER, "--gen", str(config), "--write-mtx", path], check=True, timeout=600,
                   capture_output=True)
    rows = run(["--mtx", path, "--O", str(O), "--segw", "32", "--tileK", "128", "--repeat", "2",
                "--warmup", "1", "--algo", "vcsr_mc,vcsr_mc_fp32", "--check", check,
                "--bdist", "uniform", "--csv"])
    os.remove(path)
    for name in ("vcsr_mc", "vcsr_mc_fp32"):
        assert rows[name][11] == "pass", rows[name]
        print(f"  {name}: rel_l2 {rows[name][12]}", flush=True)
