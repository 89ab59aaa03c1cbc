"""vcsrmc_spmm_noalloc (the entry point that allocates nothing) against vcsrmc_spmm_ex, through
the C ABI: bit for bit on two calls in a row, the second with a smaller input, for the launch
that converts an FP32 B into the static scratch (FP16 format) and for launches that need no
scratch; an input whose conversion exceeds the scratch is refused before anything runs; and the
call leaves the device's free memory unchanged where vcsrmc_spmm_ex allocates."""
import ctypes as C

import numpy as np
import pytest

import vcsr_mc_amd as vm
from conftest import random_csr
from gpu_util import dev, say

pytestmark = pytest.mark.gpu


def _noalloc(f, B, Cout, O, tileK=128, overwrite=False):
    import torch
    b_dtype = vm.B_F16 if B.dtype == torch.float16 else vm.B_F32
    stream = int(torch.cuda.current_stream().cuda_stream)
    return vm.lib().vcsrmc_spmm_noalloc(f.handle, B.data_ptr(), b_dtype, int(O), int(tileK),
                                        Cout.data_ptr(), vm.SPMM_OVERWRITE if overwrite else 0,
                                        stream)


def _converts(nnz, N, O, num_chunks):
    """The launcher's rule for converting an FP32 B to binary16 once per call."""
    b32 = N * O * 4
    return nnz >= 12 * N and ((nnz < 48 * num_chunks and b32 > 12 << 20) or b32 > 256 << 20)


@pytest.mark.parametrize("overwrite", [False, True])
def test_noalloc_matches_spmm_two_calls(overwrite):
    """A uniform 30,000^2 matrix with about 16 nonzeros per row and FP32 B of 128 columns
    (15 MB) takes the conversion path; the second call uses 120 columns of a 27,000-row matrix
    (13 MB: a smaller conversion, the scratch still holding the first call's halves)."""
    import torch
    for M, O, seed in ((30000, 128, 41), (27000, 120, 42)):
        rng = np.random.default_rng(seed)
        rp, c, v = random_csr(rng, M, M, nnz_per_row=16)
        B = rng.uniform(-1, 1, (M, O)).astype(np.float32)
        say("noalloc vs spmm", M, O, overwrite)
        with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, M, False, 32) as f:
            info = f.info()
            assert _converts(len(c), M, O, info["num_chunks"])
            assert M * O * 2 <= vm.NOALLOC_SCRATCH_BYTES
            dB = dev(B)
            want = torch.full((M, O), 0.5 if overwrite else 0.0, dtype=torch.float32,
                              device="cuda")
            got = want.clone()
            f.spmm(dB, want, tileK=128, overwrite=overwrite)
            assert _noalloc(f, dB, got, O, overwrite=overwrite) == vm.OK, \
                vm.lib().vcsrmc_last_error()
            torch.cuda.synchronize()
            assert torch.equal(got, want)
            assert np.array_equal(dB.cpu().numpy(), B)


@pytest.mark.parametrize("fp32,b16", [(True, False), (False, True)])
def test_noalloc_without_conversion(fp32, b16):
    """Launches that need no scratch (FP32 format, or FP16 B) give vcsrmc_spmm's result too,
    again on two calls, the second smaller."""
    import torch
    for M, N, O in ((900, 1200, 128), (300, 500, 40)):
        rng = np.random.default_rng(M + O)
        rp, c, v = random_csr(rng, M, N, density=0.01, heavy_rows=3, heavy_nnz=N // 2)
        B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
        say("noalloc no conversion", fp32, b16, M, N, O)
        with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, N, fp32, 32) as f:
            dB = dev(B).half() if b16 else dev(B)
            want = torch.zeros((M, O), dtype=torch.float32, device="cuda")
            got = torch.zeros_like(want)
            f.spmm(dB, want, tileK=64)
            assert _noalloc(f, dB, got, O, tileK=64) == vm.OK, vm.lib().vcsrmc_last_error()
            torch.cuda.synchronize()
            # split panels (the heavy rows) merge through atomics, in any order
            assert torch.allclose(got, want, rtol=1e-6, atol=1e-6)


def test_noalloc_refuses_oversized_conversion():
    """N x O binary16 values beyond the 64 MiB scratch: VCSRMC_ERR_SCRATCH, and C untouched."""
    import torch
    A = vm.generate(1, 150000)  # uniform 150,000^2, ~16 per row: converts at O = 256
    O = 256
    assert A.N * O * 2 > vm.NOALLOC_SCRATCH_BYTES
    say("noalloc oversized", A.N, A.nnz, O)
    with vm.DeviceFormat.from_device_csr(dev(A.row_ptr), dev(A.col), dev(A.val), A.M, A.N,
                                         False, 32) as f:
        assert _converts(A.nnz, A.N, O, f.info()["num_chunks"])
        dB = torch.zeros((A.N, O), dtype=torch.float32, device="cuda")
        Cout = torch.full((A.M, O), 2.0, dtype=torch.float32, device="cuda")
        assert _noalloc(f, dB, Cout, O) == vm.ERR_SCRATCH
        assert b"static scratch" in vm.lib().vcsrmc_last_error()
        torch.cuda.synchronize()
        assert bool(torch.all(Cout == 2.0))


def test_noalloc_allocates_nothing():
    """On a fresh FP16-format handle given an FP32 B that the launch converts, the first
    vcsrmc_spmm_noalloc call leaves the device's free memory where it was; the first
    vcsrmc_spmm_ex call on the same handle then allocates the N x O binary16 copy, which the
    same measurement sees.  (A first call on another handle loads the kernels beforehand, so
    code loading does not count.)"""
    import torch
    M, O = 30000, 128
    rng = np.random.default_rng(43)
    rp, c, v = random_csr(rng, M, M, nnz_per_row=16)
    B = rng.uniform(-1, 1, (M, O)).astype(np.float32)
    dB = dev(B)
    C0 = torch.zeros((M, O), dtype=torch.float32, device="cuda")
    say("noalloc allocates nothing", M, O)
    with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, M, False, 32) as warm:
        assert _converts(len(c), M, O, warm.info()["num_chunks"])
        assert _noalloc(warm, dB, C0, O) == vm.OK, vm.lib().vcsrmc_last_error()
        torch.cuda.synchronize()
    with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, M, False, 32) as f:
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        assert _noalloc(f, dB, C0, O) == vm.OK, vm.lib().vcsrmc_last_error()
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
        f.spmm(dB, C0, tileK=128)
        torch.cuda.synchronize()
        free2 = torch.cuda.mem_get_info()[0]
    assert free0 - free1 < M * O * 2, (free0, free1)
    assert free1 - free2 >= M * O * 2, (free1, free2)
