"""GPU format pipeline vs the oracle: the VCSRMC arrays built on the GPU from a device CSR must
equal, bit for bit, the oracle's (= the reference's csr_to_vcsr_mc after ordering tied rows by
ascending row id), and the committed fixtures written by the reference itself."""
import numpy as np
import pytest

import vcsr_mc_amd as vm
from conftest import random_csr
from golden_io import load_cases
from gpu_util import dev, say

pytestmark = pytest.mark.gpu


def gpu_format(rp, c, v, M, N, segw, fp32):
    with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, N, fp32, segw) as f:
        V = f.download()
    return {k: getattr(V, k) for k in ("M", "N", "segw", "bundle", "num_segments", "scale",
                                       "fp32", *vm._FMT_ARRAYS)}


def as_fmt(orc, d):
    d = dict(d)
    d["scale"] = np.float32(d["scale"])
    return orc.Format(d)


def test_golden_fixtures_bit_exact(orc):
    for case in load_cases():
        say("golden", case["name"])
        got = as_fmt(orc, gpu_format(case["row_ptr"], case["col"], case["val"], case["M"],
                                     case["N"], case["segw"], case["fp32"]))
        want = orc.canonicalize(orc.Format(case["ref"]))
        assert orc.formats_equal(got, want) == [], case["name"]


@pytest.mark.parametrize("seed", range(6))
def test_random_bit_exact(orc, seed):
    rng = np.random.default_rng(100 + seed)
    for t in range(6):
        M, N = int(rng.integers(1, 3000)), int(rng.integers(1, 3000))
        dens = float(rng.choice([0.0005, 0.003, 0.02, 0.1]))
        mag = float(rng.choice([1.0, 1e5, 3e-5]))
        rp, c, v = random_csr(rng, M, N, density=dens, mag=mag, empty_frac=0.2,
                              heavy_rows=int(rng.integers(0, 3)), heavy_nnz=int(rng.integers(0, N)))
        segw = int(rng.choice([16, 32, 48, 64]))
        fp32 = bool(rng.integers(0, 2))
        say("random", seed, t, M, N, dens, segw, fp32)
        got = as_fmt(orc, gpu_format(rp, c, v, M, N, segw, fp32))
        want = orc.build_format(rp, c, v, M, N, segw, fp32)
        assert orc.formats_equal(got, want) == [], (seed, t, M, N, segw, fp32)


@pytest.mark.parametrize("config,size,segw", [(1, 0, 32), (2, 0, 32), (3, 0, 32), (4, 0, 32),
                                              (5, 0, 32), (3, 20, 32), (4, 64, 32), (5, 12, 32),
                                              (5, 16, 16), (1, 0, 48), (2, 0, 16), (2, 0, 64),
                                              (3, 0, 16), (4, 0, 16), (4, 0, 64), (5, 0, 48)])
def test_workloads_bit_exact(orc, config, size, segw):
    """Every workload at its full benchmark size (and reduced sizes), at segw 32 and at the
    other segment widths the reference takes (16, 48, 64; 48 does not divide N, so the last
    segment is partial): the format arrays of the GPU pipeline equal the oracle's
    (src/vcsr_mc.cu:25-123) bit for bit."""
    A = vm.generate(config, size)
    fp32 = vm.WORKLOADS[config]["precision"] == "fp32"
    say("workload", config, size, A.M, A.nnz)
    got = as_fmt(orc, gpu_format(A.row_ptr, A.col, A.val, A.M, A.N, segw, fp32))
    want = orc.build_format(A.row_ptr, A.col, A.val, A.M, A.N, segw, fp32)
    assert orc.formats_equal(got, want) == []


def test_many_groups_chunked_items(orc):
    """G >= 131072: items are runs of 32 groups (src/vcsr_mc.cu:111)."""
    rng = np.random.default_rng(7)
    M = 70000
    k = rng.poisson(30, M).clip(0, M)
    rp = np.zeros(M + 1, np.int32)
    rp[1:] = np.cumsum(k)
    c = np.concatenate([np.sort(rng.choice(M, size=int(x), replace=False)) for x in k]).astype(np.int32)
    v = rng.uniform(-1, 1, c.size).astype(np.float32)
    say("chunked items", M, c.size)
    got = as_fmt(orc, gpu_format(rp, c, v, M, M, 16, False))
    want = orc.build_format(rp, c, v, M, M, 16, False)
    assert len(want["item_gbeg"]) < len(want["group_depth"]) // 16
    assert orc.formats_equal(got, want) == []


def test_upload_roundtrip(orc, rng):
    rp, c, v = random_csr(rng, 700, 900, density=0.01, empty_frac=0.1)
    want = orc.build_format(rp, c, v, 700, 900, 32, False)
    V = vm.VCSRMC(M=700, N=900, segw=32, bundle=16, num_segments=want["num_segments"],
                  scale=float(want["scale"]), fp32=False,
                  **{k: want[k] for k in vm._FMT_ARRAYS})
    say("upload roundtrip")
    with vm.DeviceFormat.from_host_format(V) as f:
        back = f.download()
        info = f.info()
    assert info["nnz"] == c.size
    got = as_fmt(orc, {k: getattr(back, k) for k in ("M", "N", "segw", "bundle", "num_segments",
                                                     "scale", "fp32", *vm._FMT_ARRAYS)})
    assert orc.formats_equal(got, want) == []


def test_build_errors():
    say("build errors")
    rp = np.array([0, 2, 3], np.int32)
    with pytest.raises(vm.VCSRMCError) as e:
        vm.DeviceFormat.from_device_csr(dev(rp), dev(np.array([3, 1, 0], np.int32)),
                                        dev(np.ones(3, np.float32)), 2, 5, False, 16)
    assert e.value.status == vm.ERR_UNSORTED
    with pytest.raises(vm.VCSRMCError) as e:
        vm.DeviceFormat.from_device_csr(dev(rp), dev(np.array([1, 1, 0], np.int32)),
                                        dev(np.ones(3, np.float32)), 2, 5, False, 16)
    assert e.value.status == vm.ERR_UNSORTED
    with pytest.raises(vm.VCSRMCError) as e:
        vm.DeviceFormat.from_device_csr(dev(rp), dev(np.array([1, 7, 0], np.int32)),
                                        dev(np.ones(3, np.float32)), 2, 5, False, 16)
    assert e.value.status == vm.ERR_CSR
    with pytest.raises(vm.VCSRMCError) as e:
        vm.DeviceFormat.from_device_csr(dev(np.array([0, 3, 2], np.int32)),
                                        dev(np.array([1, 2, 0], np.int32)),
                                        dev(np.ones(3, np.float32)), 2, 5, False, 16)
    assert e.value.status == vm.ERR_CSR
    with pytest.raises(vm.VCSRMCError) as e:
        vm.DeviceFormat.from_device_csr(dev(rp), dev(np.array([0, 1, 0], np.int32)),
                                        dev(np.ones(3, np.float32)), 2, 5, False, 24)
    assert e.value.status == vm.ERR_SEGW


def test_python_binding_checks_operands():
    """The Python binding checks sizes, element types and devices on the host, before any
    launch: a row_ptr of M elements, int64 columns, a B of N - 1 rows, a C of M - 1 rows and a
    host B are refused; the valid call then runs."""
    import torch
    say("binding operand checks")
    rp = np.array([0, 2, 3], np.int32)
    c = np.array([0, 4, 1], np.int32)
    v = np.ones(3, np.float32)
    for args in ((dev(rp[:2]), dev(c), dev(v)), (dev(rp), dev(c.astype(np.int64)), dev(v))):
        with pytest.raises(vm.VCSRMCError) as e:
            vm.DeviceFormat.from_device_csr(*args, 2, 5)
        assert e.value.status == vm.ERR_ARG
    with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), 2, 5) as f:
        C = torch.zeros((2, 8), dtype=torch.float32, device="cuda")
        ones = lambda n, where="cuda": torch.ones((n, 8), device=where)
        for B, Cout in ((ones(4), C), (ones(5), C[:1]), (ones(5, "cpu"), C)):
            with pytest.raises(vm.VCSRMCError) as e:
                f.spmm(B, Cout)
            assert e.value.status == vm.ERR_ARG
        f.spmm(ones(5), C)
        torch.cuda.synchronize()
    assert C.cpu().numpy().tolist() == [[2.0] * 8, [1.0] * 8]


def test_upload_rejects_inconsistent_arrays(orc, rng):
    rp, c, v = random_csr(rng, 100, 100, density=0.05)
    f = orc.build_format(rp, c, v, 100, 100, 16, False)
    base = dict(M=100, N=100, segw=16, bundle=16, num_segments=f["num_segments"], scale=1.0,
                fp32=False)
    arrays = {k: np.array(f[k], copy=True) for k in vm._FMT_ARRAYS}
    say("upload errors")
    for bad in ("lcol_range", "row_range", "ptr"):
        a = {k: x.copy() for k, x in arrays.items()}
        if bad == "lcol_range":
            a["lcol"][np.argmax(a["lcol"] >= 0)] = 16
        elif bad == "row_range":
            a["group_rows"][0] = 100
        else:
            a["group_ptr"][1] += 16
        with pytest.raises(vm.VCSRMCError) as e:
            vm.DeviceFormat.from_host_format(vm.VCSRMC(**base, **a))
        assert e.value.status == vm.ERR_FORMAT, bad
