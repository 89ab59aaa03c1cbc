"""Row steps of FP32 panels (v_mfma_f32_4x4x1_16b_f32 with one column per row group and step)
against the oracle, with the parity norm of the other GPU tests (tau = 1e-5 per row, C0 counted
where C starts non-zero)."""
import numpy as np
import pytest

import vcsr_mc_amd as vm
from conftest import random_csr
from gpu_util import dev, row_l1_parity, say

pytestmark = pytest.mark.gpu

TAU32 = 1e-5


@pytest.fixture
def steps_mode():
    """Sets the FP32 row-step mode for the test and restores the default afterwards."""
    def set_mode(mode):
        vm.set_fp32_row_steps(mode)
    yield set_mode
    vm.set_fp32_row_steps(vm.FP32_ROW_STEPS_AUTO)


def run(orc, rp, c, v, M, N, O, tileK=128, overwrite=False, seed=0, grouping=None):
    """One FP32 build and launch; C starts random (accumulate) or random and overwritten.
    Returns the layout info after checking every row against the oracle."""
    import torch
    rng = np.random.default_rng(seed)
    B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, O)).astype(np.float32)
    if grouping is not None:
        vm.set_row_grouping(grouping)
    try:
        with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, N, True, 32) as f:
            info = f.info()
            C = dev(C0)
            f.spmm(dev(B), C, tileK=tileK, overwrite=overwrite)
            torch.cuda.synchronize()
            Cg = C.cpu().numpy()
    finally:
        if grouping is not None:
            vm.set_row_grouping(vm.ROW_GROUPING_AUTO)
    R, L1 = orc.spmm_csr(rp, c, v, M, B, mode=0, scale=info["scale"])
    touched = np.diff(rp) > 0
    if overwrite:
        # rows A touches are A.B; the others keep C0
        R = np.where(touched[:, None], R, C0.astype(np.float64))
    else:
        R = R + C0.astype(np.float64)
        L1 = L1 + np.abs(C0.astype(np.float64)).sum(axis=1)
    ok, worst, r = row_l1_parity(Cg, R, L1, TAU32)
    assert ok, f"row {r}: error / bound = {worst:.3g} ({info})"
    if overwrite:
        assert np.array_equal(Cg[~touched], C0[~touched])
    return info


@pytest.mark.parametrize("O", [128, 100, 7])
@pytest.mark.parametrize("overwrite", [False, True])
def test_uniform_takes_row_steps_by_default(orc, steps_mode, O, overwrite):
    """A uniform random 4096^2 FP32 matrix (16 per row) takes row steps in the default mode,
    all of its panels or nearly; tile steps only in mode 0, with the same results."""
    rng = np.random.default_rng(3)
    rp, c, v = random_csr(rng, 4096, 4096, nnz_per_row=16)
    say("row steps uniform default", O, overwrite)
    info = run(orc, rp, c, v, 4096, 4096, O, overwrite=overwrite, seed=O)
    assert info["num_row_step_batches"] >= info["num_panels"], info
    steps_mode(vm.FP32_ROW_STEPS_OFF)
    say("row steps uniform off", O, overwrite)
    info = run(orc, rp, c, v, 4096, 4096, O, overwrite=overwrite, seed=O)
    assert info["num_row_step_batches"] == 0, info


@pytest.mark.parametrize("tileK", [16, 32, 64, 128])
def test_all_tile_widths(orc, steps_mode, tileK):
    """Every O tile width with row steps for every panel (mode 2), O past the vector width."""
    steps_mode(vm.FP32_ROW_STEPS_ALWAYS)
    rng = np.random.default_rng(tileK)
    rp, c, v = random_csr(rng, 3000, 2500, nnz_per_row=9, empty_frac=0.1)
    say("row steps tileK", tileK)
    info = run(orc, rp, c, v, 3000, 2500, 133, tileK=tileK, seed=tileK)
    assert info["num_row_step_batches"] > 0


def band(M, N, bw):
    rows, cols = [], []
    for r in range(M):
        lo, hi = max(0, r - bw), min(N, r + bw + 1)
        rows.append(np.full(hi - lo, r))
        cols.append(np.arange(lo, hi))
    rows = np.concatenate(rows)
    cols = np.concatenate(cols).astype(np.int32)
    rp = np.zeros(M + 1, np.int32)
    rp[1:] = np.cumsum(np.bincount(rows, minlength=M))
    return rp, cols


@pytest.mark.parametrize("overwrite", [False, True])
def test_forced_on_every_structure(orc, steps_mode, overwrite):
    """Mode 2 on structures the default leaves on tiles: a dense band (every row group reads
    every column), heavy rows cut into several heavy units (merged through atomics), rows
    grouped into panels by shared columns (a row map), a single column, and mostly empty
    rows."""
    steps_mode(vm.FP32_ROW_STEPS_ALWAYS)
    rng = np.random.default_rng(11)
    cases = []
    rp, c = band(2048, 2048, 20)
    cases.append(("band", rp, c, 2048, 2048, None))
    rp, c, _ = random_csr(rng, 640, 30000, nnz_per_row=4, heavy_rows=3, heavy_nnz=9000)
    cases.append(("heavy rows", rp, c, 640, 30000, None))
    n = 24
    idx = np.arange(n ** 3).reshape(n, n, n)
    rows, cols = [], []
    for dz in (-1, 0, 1):
        for dy in (-1, 0, 1):
            for dx in (-1, 0, 1):
                src = idx[max(0, -dz):n - max(0, dz), max(0, -dy):n - max(0, dy),
                          max(0, -dx):n - max(0, dx)]
                dst = idx[max(0, dz):n - max(0, -dz), max(0, dy):n - max(0, -dy),
                          max(0, dx):n - max(0, -dx)]
                rows.append(src.ravel())
                cols.append(dst.ravel())
    rows, cols = np.concatenate(rows), np.concatenate(cols)
    order = np.lexsort((cols, rows))
    rows, cols = rows[order], cols[order].astype(np.int32)
    rp = np.zeros(n ** 3 + 1, np.int32)
    rp[1:] = np.cumsum(np.bincount(rows, minlength=n ** 3))
    cases.append(("stencil grouped", rp, cols, n ** 3, n ** 3, vm.ROW_GROUPING_ALWAYS))
    rp = np.arange(0, 1001, dtype=np.int32)
    cases.append(("one column", rp, np.zeros(1000, np.int32), 1000, 1, None))
    rp, c, _ = random_csr(rng, 5000, 5000, nnz_per_row=5, empty_frac=0.9)
    cases.append(("mostly empty", rp, c, 5000, 5000, None))
    for i, (name, rp, c, M, N, grouping) in enumerate(cases):
        v = rng.uniform(-1, 1, c.size).astype(np.float32)
        say("row steps forced", name, overwrite)
        info = run(orc, rp, c, v, M, N, 64, overwrite=overwrite, seed=i, grouping=grouping)
        assert info["num_row_step_batches"] > 0, (name, info)
        if name == "heavy rows":
            assert info["num_split_panels"] > 0, info
        if name == "stencil grouped":
            assert info["row_grouped"] == 1, info


def test_power_law_mixes_units(orc, steps_mode):
    """The power-law workload matrix in FP32 at reduced size: hub panels stay on tiles, the
    others take row steps, in one launch; the whole product against the oracle."""
    A = vm.generate(2, 8000)
    say("row steps power-law mixed", A.M, A.nnz)
    info = run(orc, A.row_ptr, A.col, A.val, A.M, A.N, 128, seed=5)
    assert 0 < info["num_row_step_batches"], info
