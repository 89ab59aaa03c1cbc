"""GPU product against the reference's own kernels on the same inputs.

oracle/_ref holds MuuSeoTia/VCSR_MC's src/vcsr_mc.cu compiled for this GPU from its sources
(oracle/Makefile).  Each case runs the reference's path (csr_to_vcsr_mc, upload_vcsr_mc_device,
run_vcsr_mc_spmm_gpu: kernels vcsr_mc / vcsr_mc_fp32, src/vcsr_mc.cu:143-394) and this library's
on the same A and FP32 B, both from C = 0, and checks, per row r, with N_r = sum |a||b| of the
(FP16-quantised, for vcsr_mc) operands and tau = 1e-5 (FP32) or 2e-3 (FP16):
    ||C_ref[r] - R[r]||_1 <= tau N_r,   ||C_ours[r] - R[r]||_1 <= tau N_r,
    ||C_ours[r] - C_ref[r]||_1 <= 2 tau N_r,
with R the oracle's double-precision product -- so the oracle is pinned against the reference's
own GPU results too.  The two differ only in the order of the FP32 sums."""
import numpy as np
import pytest

import vcsr_mc_amd as vm
from conftest import random_csr
from gpu_util import dev, say

pytestmark = pytest.mark.gpu

TAU = {True: 1e-5, False: 2e-3}


def both(orc, rp, c, v, M, N, B, fp32, segw, tileK):
    import torch
    O = B.shape[1]
    dB = dev(B.astype(np.float32))
    C_ref = torch.zeros((M, O), dtype=torch.float32, device="cuda")
    C_ours = torch.zeros_like(C_ref)
    torch.cuda.synchronize()
    orc.ref_spmm_gpu(rp, c, v, M, N, dB.data_ptr(), O, C_ref.data_ptr(), segw=segw, tileK=tileK,
                     fp32=fp32)
    with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, N, fp32, segw) as f:
        f.spmm(dB, C_ours, tileK=tileK)
        scale = f.info()["scale"]
    torch.cuda.synchronize()
    a, b = C_ref.cpu().numpy(), C_ours.cpu().numpy()
    del C_ref, C_ours
    tau = TAU[fp32]
    mode = 0 if fp32 else 1
    # the oracle's row check: the rows of spmm_csr (same sums) against each C, on all cores
    err_a, L1 = orc.spmm_check(rp, c, v, M, B, a, mode=mode, scale=scale)
    err_b, _ = orc.spmm_check(rp, c, v, M, B, b, mode=mode, scale=scale)
    err_ab = np.abs(b.astype(np.float64) - a).sum(axis=1)
    for name, err, t in (("reference kernel vs oracle", err_a, tau), ("ours vs oracle", err_b, tau),
                         ("ours vs reference kernel", err_ab, 2 * tau)):
        ratio = err / (t * L1 + 1e-30)
        row = int(np.argmax(ratio)) if ratio.size else -1
        assert np.all(err <= t * L1 + 1e-30), f"{name}: row {row}, error / bound = {ratio[row]:.3g}"


@pytest.fixture
def ref(orc):
    if not orc.ref_available():
        pytest.skip("oracle/_ref (the reference's build) is not present")
    return orc


@pytest.mark.parametrize("fp32", [False, True])
@pytest.mark.parametrize("segw,tileK,O", [(16, 32, 64), (32, 128, 128), (64, 128, 100),
                                          (48, 64, 33)])
def test_random_against_reference_kernel(ref, fp32, segw, tileK, O):
    rng = np.random.default_rng(segw * 7 + O + fp32)
    M, N = 1500, 1300
    rp, c, v = random_csr(rng, M, N, nnz_per_row=9, heavy_rows=3, heavy_nnz=700,
                          empty_frac=0.1)
    B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
    say("reference kernel: random", fp32, segw, tileK, O)
    both(ref, rp, c, v, M, N, B, fp32, segw, tileK)


@pytest.mark.parametrize("config,size,fp32", [(1, 2048, True), (2, 6000, False), (2, 6000, True),
                                              (3, 18, True), (3, 18, False), (4, 96, False),
                                              (5, 13, False), (1, 0, True), (2, 0, False),
                                              (3, 0, True), (4, 0, False), (5, 0, False)])
def test_workloads_against_reference_kernel(ref, config, size, fp32):
    """The five workload generators at reduced sizes and at their full benchmark sizes (in the
    precision each is configured for), at each workload's O and segw 32."""
    A = vm.generate(config, size)
    O = vm.WORKLOADS[config]["O"]
    B = vm.dense(A.N, O, seed=vm.SEED_BASE + 100 + config, fp16_exact=not fp32)
    say("reference kernel: workload", config, size, fp32, A.M, A.nnz, O)
    both(ref, A.row_ptr, A.col, A.val, A.M, A.N, B, fp32, 32, 128)
