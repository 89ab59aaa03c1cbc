"""The drop-in boundary, without a GPU.

* The reference's own driver (src/main.cpp) and hipSPARSE file (src/kernels.cu), compiled from
  its sources against this repository's include/ and linked with libvcsrmc.so
  (oracle/_ref/spmm_vcsr_dropin, built by `make -C oracle ref`): every VCSR-MC, format and
  reordering function it calls resolves to libvcsrmc.so, and its Matrix Market path -- which runs
  before the driver touches the GPU -- goes through include/mmio.hpp and include/csr.hpp.
* include/mmio.hpp + include/csr.hpp against the reference's reader on committed fixtures
  (tests/golden/mtx_golden.json: the CSR arrays, or the error text, of 45 files).
* The C++ upload_vcsr_mc_device refuses format vectors whose lengths disagree."""
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
PKG = os.path.join(ROOT, "vcsr_mc_amd")
REF_SRC = "/root/reference/src/main.cpp"
DROPIN = os.path.join(ROOT, "oracle", "_ref", "spmm_vcsr_dropin")
GOLDEN = os.path.join(ROOT, "tests", "golden", "mtx_golden.json")

DROPIN_FUNCS = ("half_scale(CSR const&)", "csr_to_vcsr_mc(CSR const&, bool, int)",
                "upload_vcsr_mc_device(VCSRMC const&)",
                "run_vcsr_mc_spmm_gpu(VCSRMC const&, float const*, int, int, float*, "
                "ihipStream_t*, float&)",
                "destroy_vcsr_mc_device(ihipStream_t*)", "rcm_column_order(CSR const&)")


def _nm(path, *flags):
    return subprocess.run(["nm", "-C", *flags, path], capture_output=True, text=True,
                          check=True).stdout


@pytest.fixture(scope="module")
def dropin():
    if not os.path.exists(REF_SRC):
        pytest.skip("reference sources absent")
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), DROPIN], check=True,
                   capture_output=True)
    return DROPIN


def test_reference_driver_links_against_library(dropin):
    undefined = _nm(dropin, "--undefined-only")
    defined = _nm(os.path.join(PKG, "libvcsrmc.so"), "-D", "--defined-only")
    for f in DROPIN_FUNCS:
        assert f in undefined, f
        assert f in defined, f
    assert "apply_column_permutation(CSR&" in undefined
    assert "apply_column_permutation(CSR&" in defined
    libs = subprocess.run(["ldd", dropin], capture_output=True, text=True).stdout
    assert os.path.join("vcsr_mc_amd", "libvcsrmc.so") in libs.replace("../../", "")


def test_reference_driver_reads_mtx_through_include(dropin, tmp_path):
    """The reference's driver reports this repository's reader errors (a GPU is touched only
    after the CSR is built, main.cpp:150-157)."""
    for body, msg in ((
            "%%MatrixMarket matrix coordinate real general\n2 2 2\n1 2 1\n1 2 3\n",
            "Duplicate MTX coordinates"),
            ("%%MatrixMarket matrix coordinate real general\n2 2 1\n1 1 3.0x\n",
             "Extra fields in MTX entry"),
            ("%%MatrixMarket matrix coordinate real hermitian\n1 1 0\n",
             "Unsupported MTX symmetry: hermitian")):
        f = tmp_path / "a.mtx"
        f.write_text(body)
        r = subprocess.run([dropin, "--mtx", str(f)], capture_output=True, text=True, timeout=60)
        assert r.returncode == 2 and msg in r.stderr, r.stderr
    r = subprocess.run([dropin, "--help"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "Usage: spmm_vcsr" in r.stdout


@pytest.fixture(scope="module")
def mtx_dump(tmp_path_factory):
    """oracle/mtx_dump.cpp built against this repository's include/ (header-only reader)."""
    exe = tmp_path_factory.mktemp("mtx") / "mtx_dump"
    subprocess.run(["g++", "-O1", "-std=c++17", "-Wall", "-Werror", f"-I{INC}",
                    os.path.join(ROOT, "oracle", "mtx_dump.cpp"), "-o", str(exe)], check=True)
    return str(exe)


def test_mtx_reader_matches_reference_fixtures(mtx_dump, tmp_path):
    cases = json.load(open(GOLDEN))
    assert len(cases) >= 40
    n_ok = 0
    for name, case in sorted(cases.items()):
        path = tmp_path / f"{name}.mtx"
        with open(path, "w", newline="") as fh:
            fh.write(case["body"])
        got = subprocess.run([mtx_dump, str(path)], capture_output=True, text=True,
                             check=True).stdout
        assert got == case["reference"], name
        n_ok += case["reference"].startswith("OK")
    assert n_ok >= 12  # valid inputs as well as errors


def test_mtx_reader_missing_file(mtx_dump, tmp_path):
    got = subprocess.run([mtx_dump, str(tmp_path / "none.mtx")], capture_output=True, text=True,
                         check=True).stdout
    assert got == f"ERR Failed to open MTX: {tmp_path / 'none.mtx'}\n"


def test_cpp_upload_refuses_inconsistent_vectors(tmp_path):
    src = tmp_path / "u.cpp"
    src.write_text(r'''
#include <cstdio>
#include <stdexcept>
#include "vcsr_formats.hpp"
int main() {
    VCSRMC V;
    V.M = V.N = 16; V.segw = 16; V.num_segments = 1;
    V.group_depth = {1}; V.group_ptr = {0, 16}; V.group_seg_base = {0};
    V.group_rows.assign(15, 0);  // 16 needed
    V.lcol.assign(16, -1); V.val.assign(16, 0.f); V.item_gbeg = {0}; V.item_gend = {1};
    try { upload_vcsr_mc_device(V); } catch (const std::runtime_error& e) {
        std::printf("%s\n", e.what()); return 0; }
    return 1;
}
''')
    exe = tmp_path / "u"
    subprocess.run(["/opt/rocm/bin/amdclang++", "-std=c++17", "-D__HIP_PLATFORM_AMD__",
                    "-I/opt/rocm/include", f"-I{INC}", str(src), f"-L{PKG}", "-lvcsrmc",
                    f"-Wl,-rpath,{PKG}", "-L/opt/rocm/lib", "-lamdhip64", "-o", str(exe)],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "differ in length" in r.stdout, (r.stdout, r.stderr)
