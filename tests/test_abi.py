"""The C ABI libraries load on a machine without a GPU and export every function their headers
declare; the C++ drop-in surface exports the reference's five functions.  No compute calls."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")


def declared(header):
    text = open(os.path.join(INC, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vcsrmc_\w+)\s*\(", text)))


@pytest.mark.parametrize("header,lib", [("vcsrmc.h", "libvcsrmc.so"),
                                        ("vcsrmc_bench.h", "libvcsrmc_bench.so")])
def test_exports_every_declared_symbol(header, lib):
    path = os.path.join(ROOT, "vcsr_mc_amd", lib)
    assert os.path.exists(path), f"{lib} not built"
    L = ctypes.CDLL(path)
    names = declared(header)
    assert names
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_cpp_dropin_symbols():
    path = os.path.join(ROOT, "vcsr_mc_amd", "libvcsrmc.so")
    out = subprocess.run(["nm", "-DC", "--defined-only", path], capture_output=True, text=True,
                         check=True).stdout
    for sig in ("half_scale(CSR const&)",
                "csr_to_vcsr_mc(CSR const&, bool, int)",
                "upload_vcsr_mc_device(VCSRMC const&)",
                "run_vcsr_mc_spmm_gpu(VCSRMC const&, float const*, int, int, float*, "
                "ihipStream_t*, float&)",
                "destroy_vcsr_mc_device(ihipStream_t*)"):
        assert sig in out, sig


def test_status_strings_without_gpu():
    L = ctypes.CDLL(os.path.join(ROOT, "vcsr_mc_amd", "libvcsrmc.so"))
    L.vcsrmc_status_string.restype = ctypes.c_char_p
    assert b"tileK" in L.vcsrmc_status_string(3)
    assert b"segw" in L.vcsrmc_status_string(2)


def test_no_oracle_in_product():
    """The product library must not link or name the oracle."""
    for lib in ("libvcsrmc.so",):
        path = os.path.join(ROOT, "vcsr_mc_amd", lib)
        deps = subprocess.run(["ldd", path], capture_output=True, text=True).stdout
        assert "oracle" not in deps
        syms = subprocess.run(["nm", "-D", path], capture_output=True, text=True).stdout
        assert "orc_" not in syms and "ref_build" not in syms


@pytest.mark.parametrize("field,delta", [("group_ptr", -1), ("group_seg_base", 1),
                                          ("group_rows", -16), ("lcol", -1), ("item_gend", 1)])
def test_upload_refuses_short_arrays_without_gpu(field, delta):
    """from_host_format checks every array length against the sizes the format implies before a
    handle exists or anything is copied (the C ABI reads those sizes from each pointer)."""
    import numpy as np

    import vcsr_mc_amd as vm
    G, nval, ni = 2, 64, 1
    V = vm.VCSRMC(M=32, N=32, segw=16, num_segments=2,
                  group_ptr=np.array([0, 32, 64], np.int32), group_depth=np.array([2, 2], np.int32),
                  group_seg_base=np.zeros(G, np.int32), group_rows=np.zeros(16 * G, np.int32),
                  lcol=np.zeros(nval, np.int32), val=np.zeros(nval, np.float32),
                  item_gbeg=np.zeros(ni, np.int32), item_gend=np.ones(ni, np.int32))
    a = getattr(V, field)
    setattr(V, field, np.zeros(len(a) + delta, np.int32))
    with pytest.raises(vm.VCSRMCError) as e:
        vm.DeviceFormat.from_host_format(V)
    assert e.value.status == vm.ERR_FORMAT and field in str(e.value)


def test_fp32_row_steps_mode_checked_without_gpu():
    """vcsrmc_set_fp32_row_steps accepts 0, 1 and 2 and refuses anything else before any device
    work; the default (1) is restored."""
    import vcsr_mc_amd as vm
    for mode in (vm.FP32_ROW_STEPS_OFF, vm.FP32_ROW_STEPS_ALWAYS, vm.FP32_ROW_STEPS_AUTO):
        vm.set_fp32_row_steps(mode)
    for bad in (-1, 3):
        with pytest.raises(vm.VCSRMCError) as e:
            vm.set_fp32_row_steps(bad)
        assert e.value.status == vm.ERR_ARG
    vm.set_fp32_row_steps(vm.FP32_ROW_STEPS_AUTO)


def test_row_grouping_mode_checked_without_gpu():
    """vcsrmc_set_row_grouping accepts 0, 1 and 2 and refuses anything else before any device
    work; the default (1) is restored."""
    import vcsr_mc_amd as vm
    for mode in (vm.ROW_GROUPING_OFF, vm.ROW_GROUPING_ALWAYS, vm.ROW_GROUPING_AUTO):
        vm.set_row_grouping(mode)
    for bad in (-1, 3):
        with pytest.raises(vm.VCSRMCError) as e:
            vm.set_row_grouping(bad)
        assert e.value.status == vm.ERR_ARG
    vm.set_row_grouping(vm.ROW_GROUPING_AUTO)
