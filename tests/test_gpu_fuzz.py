"""Seeded random inputs through the whole device path -- format build, execution layout in each
row-order mode and FP32 row-step mode, SpMM in both launch modes -- against the oracle with the parity gate of
test_gpu_spmm.py: uniform and Poisson rows with heavy rows and empty rows, bands, 2D 5-point
grids and dense blocks at random block columns (light units in column order); FP16 / FP32
formats, FP16 or FP32 B, segw 16-64, tileK 16-128, O from 1 to 256.  Rows A does not touch must
keep C's values."""
import numpy as np
import pytest

import vcsr_mc_amd as vm
from conftest import random_csr
from gpu_util import dev, row_l1_parity, say

pytestmark = pytest.mark.gpu

TAU = {True: 1e-5, False: 2e-3}


def _band(rng, M, N, bw):
    rows = [np.arange(max(0, min(r, N - 1) - bw), min(N, min(r, N - 1) + bw + 1))
            for r in range(M)]
    rp = np.zeros(M + 1, np.int32)
    rp[1:] = np.cumsum([len(x) for x in rows])
    c = np.concatenate(rows).astype(np.int32)
    return rp, c, rng.uniform(-1, 1, c.size).astype(np.float32)


def _grid5(rng, g):
    M = g * g
    idx = np.arange(M)
    x, y = idx % g, idx // g
    cols = [np.where((x + dx >= 0) & (x + dx < g) & (y + dy >= 0) & (y + dy < g),
                     x + dx + g * (y + dy), -1)
            for dx, dy in ((0, -1), (-1, 0), (0, 0), (1, 0), (0, 1))]
    C5 = np.sort(np.stack(cols, 1), axis=1)
    keep = C5 >= 0
    rp = np.zeros(M + 1, np.int32)
    rp[1:] = np.cumsum(keep.sum(1))
    c = C5[keep].astype(np.int32)
    return rp, c, rng.uniform(-1, 1, c.size).astype(np.float32)


def _blocks(rng, M, N, b, per_row):
    """Dense b x b blocks at `per_row` distinct random block columns of every block row."""
    nbc = max(1, N // b)
    rows = []
    for br in range((M + b - 1) // b):
        bc = np.sort(rng.choice(nbc, size=min(per_row, nbc), replace=False))
        cols = (bc[:, None] * b + np.arange(b)[None, :]).ravel()
        cols = cols[cols < N]
        rows += [cols] * min(b, M - br * b)
    rp = np.zeros(M + 1, np.int32)
    rp[1:] = np.cumsum([len(x) for x in rows])
    c = np.concatenate(rows).astype(np.int32)
    return rp, c, rng.uniform(-1, 1, c.size).astype(np.float32)


@pytest.mark.parametrize("seed", range(4))
def test_fuzz_all_row_orders(orc, seed):
    import torch
    rng = np.random.default_rng(30000 + seed)
    rng_steps = np.random.default_rng(40000 + seed)  # its own stream: the cases stay as they were
    try:
        for t in range(50):
            mode = int(rng.integers(0, 3))
            vm.set_row_grouping(mode)
            steps = int(rng_steps.integers(0, 3))
            vm.set_fp32_row_steps(steps)
            M, N = int(rng.integers(1, 5000)), int(rng.integers(1, 5000))
            kind = int(rng.integers(0, 5))
            if kind == 0:
                rp, c, v = random_csr(rng, M, N, density=float(rng.choice([0.0005, 0.003, 0.02])),
                                      empty_frac=float(rng.uniform(0, 0.5)))
            elif kind == 1:
                rp, c, v = random_csr(rng, M, N, nnz_per_row=float(rng.uniform(0.5, 12)),
                                      heavy_rows=int(rng.integers(0, 4)),
                                      heavy_nnz=int(rng.integers(1, N + 1)))
            elif kind == 2:
                rp, c, v = _band(rng, M, N, int(rng.integers(0, 20)))
            elif kind == 3:
                g = int(rng.integers(2, 60))
                M = N = g * g
                rp, c, v = _grid5(rng, g)
            else:
                rp, c, v = _blocks(rng, M, N, int(rng.choice([4, 8, 16, 32])),
                                   int(rng.integers(1, 6)))
            fp32 = bool(rng.integers(0, 2))
            segw = int(rng.choice([16, 32, 48, 64]))
            tileK = int(rng.choice([16, 32, 64, 128]))
            O = int(rng.choice([1, 5, 8, 33, 64, 100, 128, 200, 256]))
            overwrite = bool(rng.integers(0, 2))
            b16 = (not fp32) and bool(rng.integers(0, 2))
            B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
            if not fp32:
                B = B.astype(np.float16).astype(np.float32)
            C0 = rng.uniform(-1, 1, (M, O)).astype(np.float32)
            say("fuzz", seed, t, mode, steps, kind, M, N, c.size, fp32, segw, tileK, O,
                overwrite, b16)
            with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, N, fp32, segw) as f:
                scale = f.info()["scale"]
                dB = dev(B).half() if b16 else dev(B)
                dC = dev(C0)
                f.spmm(dB, dC, tileK=tileK, overwrite=overwrite)
                torch.cuda.synchronize()
                Cg = dC.cpu().numpy()
            R, L1 = orc.spmm_csr(rp, c, v, M, B, mode=0 if fp32 else 1, scale=scale)
            touched = np.diff(rp) > 0
            base = C0.astype(np.float64).copy()
            if overwrite:
                base[touched] = 0.0
            ok, worst, row = row_l1_parity(Cg, R + base, L1 + np.abs(base).sum(axis=1),
                                           TAU[fp32])
            assert ok, f"case {t}: row {row}: error / bound = {worst:.3g}"
            assert np.array_equal(Cg[~touched], C0[~touched]), f"case {t}: untouched rows"
    finally:
        vm.set_row_grouping(vm.ROW_GROUPING_AUTO)
        vm.set_fp32_row_steps(vm.FP32_ROW_STEPS_AUTO)
