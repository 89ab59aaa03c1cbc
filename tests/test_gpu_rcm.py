"""GPU column reordering (vcsrmc_rcm_order / vcsrmc_apply_column_permutation) against the
oracle's restatement of include/reorder.hpp:17-108 and the committed fixtures made by the
reference's compiled header: positions, relabelled CSR and permuted B bit for bit."""
import os

import numpy as np
import pytest

import vcsr_mc_amd as vm
from conftest import random_csr
from gpu_util import dev, say, row_l1_parity
from golden_io import banded, csr_from_edges, grid5

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "rcm_golden.npz")


def gpu_rcm(rp, col, M, N):
    import torch
    pos = torch.empty(max(N, 1), dtype=torch.int32, device="cuda")
    vm.rcm_order_device(dev(rp), dev(col), M, N, pos)
    torch.cuda.synchronize()
    return pos[:N].cpu().numpy()


def gpu_apply(rp, col, val, M, N, pos, B, O):
    import torch
    ci, vv = dev(col), dev(val)
    Bd = dev(np.ascontiguousarray(B, np.float32).reshape(-1))
    Bo = torch.empty_like(Bd)
    vm.apply_column_permutation_device(dev(rp), ci, vv, M, N, dev(pos), Bd, Bo, O)
    torch.cuda.synchronize()
    return ci.cpu().numpy(), vv.cpu().numpy(), Bo.cpu().numpy().reshape(N, O)


def test_rcm_fixtures_gpu():
    gold = np.load(GOLDEN)
    for name in gold["cases"]:
        rp, col = gold[f"{name}/row_ptr"], gold[f"{name}/col"]
        M, N = (int(x) for x in gold[f"{name}/shape"])
        say("rcm fixture", name, M, N, col.size)
        pos = gpu_rcm(rp, col, M, N)
        assert np.array_equal(pos, gold[f"{name}/position"]), name
        B = gold[f"{name}/B"]
        c2, v2, B2 = gpu_apply(rp, col, gold[f"{name}/val"], M, N, pos, B, B.shape[1])
        assert np.array_equal(c2, gold[f"{name}/new_col"]), name
        assert np.array_equal(v2, gold[f"{name}/new_val"]), name
        assert np.array_equal(B2, gold[f"{name}/new_B"]), name


def test_rcm_adversarial_hub_gpu():
    """A 2000-child group sorted by adversarial degrees: work-group partition passes, then the
    heapsort fallback on a 1960-element range, must give the reference's order."""
    from golden_io import adversary_hub
    gold = np.load(GOLDEN)
    rp, col, N = adversary_hub(gold["hub2000/keys"])
    say("rcm adversarial hub", N, col.size)
    assert np.array_equal(gpu_rcm(rp, col, N, N), gold["hub2000/position"])


def test_rcm_random_gpu(orc):
    rng = np.random.default_rng(11)
    for t in range(40):
        M, N = int(rng.integers(1, 2000)), int(rng.integers(1, 2000))
        rp, col, val = random_csr(rng, M, N, nnz_per_row=float(rng.uniform(0, 10)),
                                  heavy_rows=int(rng.integers(0, 4)), heavy_nnz=400,
                                  empty_frac=float(rng.uniform(0, 0.5)))
        say("rcm random", t, M, N, col.size)
        pos = gpu_rcm(rp, col, M, N)
        assert np.array_equal(pos, orc.rcm_order(rp, col, M, N)), t


@pytest.mark.parametrize("config,size", [(1, 2048), (2, 0), (3, 40), (4, 512), (5, 14),
                                         (1, 0), (3, 0), (4, 0), (5, 0)])
def test_rcm_workloads_gpu(orc, config, size):
    """Column positions and the permuted CSR and B equal the oracle's element for element, on
    reduced workloads and on all five at their full benchmark sizes."""
    A = vm.generate(config, size)
    say("rcm workload", config, size, A.M, A.N, A.nnz)
    pos = gpu_rcm(A.row_ptr, A.col, A.M, A.N)
    assert np.array_equal(pos, orc.rcm_order(A.row_ptr, A.col, A.M, A.N))
    O = 4
    B = np.random.default_rng(config).uniform(-1, 1, (A.N, O)).astype(np.float32)
    c2, v2, B2 = gpu_apply(A.row_ptr, A.col, A.val, A.M, A.N, pos, B, O)
    e2, w2, D2 = orc.apply_column_permutation(A.row_ptr, A.col, A.val, A.M, A.N, pos, B, O)
    assert np.array_equal(c2, e2) and np.array_equal(v2, w2) and np.array_equal(B2, D2)


@pytest.mark.parametrize("N", [1100, 2000, 20000])
def test_rcm_path_gpu(N):
    """Deep walks: the levels run inside one work-group.  Vertex 0 has the lowest (degree, id),
    the walk is 0, 1, ..., N - 1, so position[c] = N - 1 - c.  Long union-find chains here once
    left non-root parents behind (a path-halving store landing after the final root)."""
    rp, col = banded(N, 1)
    say("rcm path", N)
    assert np.array_equal(gpu_rcm(rp, col, N, N), N - 1 - np.arange(N))


@pytest.mark.parametrize("shape", [("band", 100000, 10), ("grid", 400, 400), ("grid", 90, 700)])
def test_rcm_banded_and_grid_gpu(orc, shape):
    """Frontiers that grow past one work-group (grids: anti-diagonals up to 400 vertices with
    up to 5 edges each) switch between the work-group levels and the multi-kernel levels."""
    kind, a, b = shape
    rp, col = banded(a, b) if kind == "band" else grid5(a, b)
    N = rp.size - 1
    say("rcm", kind, a, b, N, col.size)
    assert np.array_equal(gpu_rcm(rp, col, N, N), orc.rcm_order(rp, col, N, N))


def test_rcm_structured_sweep_gpu(orc):
    """Shapes the random matrices rarely make: paths glued to hubs (deep walks next to wide
    levels, child groups beyond the work-group sort), many small components, grids with a few
    long-range edges, and rows beyond N with isolated columns."""
    for t in range(24):
        rng = np.random.default_rng(900 + t)
        kind = t % 4
        if kind == 0:
            N = int(rng.integers(2, 20000))
            perm = rng.permutation(N)
            cut = np.sort(rng.choice(np.arange(1, N), size=min(N - 1, int(rng.integers(0, 12))),
                                     replace=False))
            e = [(a, b) for seg in np.split(perm, cut) for a, b in zip(seg[:-1], seg[1:])]
            for _ in range(int(rng.integers(0, 4))):
                hub = int(rng.integers(0, N))
                e += [(hub, int(x)) for x in rng.choice(N, size=min(N, int(rng.integers(1, 3000))),
                                                        replace=False)]
            e += [(b, a) for a, b in e]
            M = N
            rp, col = csr_from_edges(M, N, e)
        elif kind == 1:
            N = int(rng.integers(1, 20000))
            e, start = [], 0
            while start < N:
                ids = np.arange(start, min(N, start + int(rng.integers(1, 50))))
                start += len(ids)
                for _ in range(2 * len(ids)):
                    a, b = int(rng.choice(ids)), int(rng.choice(ids))
                    e += [(a, b), (b, a)]
            M = N
            rp, col = csr_from_edges(M, N, e)
        elif kind == 2:
            rp, col = grid5(int(rng.integers(1, 250)), int(rng.integers(1, 250)))
            M = N = rp.size - 1
            e = [(r, int(c)) for r in range(M) for c in col[rp[r]:rp[r + 1]]]
            e += [(int(rng.integers(0, N)), int(rng.integers(0, N)))
                  for _ in range(int(rng.integers(1, 40)))]
            rp, col = csr_from_edges(M, N, e)
        else:
            N = int(rng.integers(1, 3000))
            M = N + int(rng.integers(0, 3000))
            rp, col, _ = random_csr(rng, M, N, nnz_per_row=float(rng.uniform(0, 2)),
                                    empty_frac=0.5)
        say("rcm structured", t, kind, M, N, col.size)
        assert np.array_equal(gpu_rcm(rp, col, M, N), orc.rcm_order(rp, col, M, N)), t


def test_rcm_no_nonzeros_gpu():
    # every column isolated: the order is 0..N-1, so position[c] = N - 1 - c
    N = 37
    pos = gpu_rcm(np.zeros(6, np.int32), np.zeros(0, np.int32), 5, N)
    assert np.array_equal(pos, N - 1 - np.arange(N))


def test_rcm_errors_gpu():
    import torch
    rp = np.array([0, 2, 3], np.int32)
    col = np.array([0, 5, 1], np.int32)
    pos = torch.empty(4, dtype=torch.int32, device="cuda")
    with pytest.raises(vm.VCSRMCError) as e:
        vm.rcm_order_device(dev(rp), dev(col), 2, 4, pos)  # column 5 >= N
    assert e.value.status == vm.ERR_CSR
    col = np.array([0, 1, 1], np.int32)
    with pytest.raises(vm.VCSRMCError) as e:  # not a permutation
        vm.apply_column_permutation_device(dev(rp), dev(col), dev(np.ones(3, np.float32)), 2, 4,
                                           dev(np.array([0, 0, 1, 2], np.int32)))
    assert e.value.status == vm.ERR_ARG
    with pytest.raises(vm.VCSRMCError) as e:  # a row holding column 0 twice
        vm.apply_column_permutation_device(dev(np.array([0, 2], np.int32)),
                                           dev(np.array([0, 0], np.int32)),
                                           dev(np.ones(2, np.float32)), 1, 4,
                                           dev(np.array([3, 2, 1, 0], np.int32)))
    assert e.value.status == vm.ERR_UNSORTED


def test_rcm_then_spmm_gpu(orc):
    """C = (A P)(P^T B) through the VCSR-MC kernels equals A B (FP32 tolerance)."""
    import torch
    A = vm.generate(2, 3000)
    say("rcm then spmm", A.M, A.N, A.nnz)
    O = 64
    B = vm.dense(A.N, O, 5)
    pos = gpu_rcm(A.row_ptr, A.col, A.M, A.N)
    c2, v2, B2 = gpu_apply(A.row_ptr, A.col, A.val, A.M, A.N, pos, B, O)
    with vm.DeviceFormat.from_device_csr(dev(A.row_ptr), dev(c2), dev(v2), A.M, A.N,
                                         fp32=True, segw=32) as f:
        Cd = torch.zeros((A.M, O), dtype=torch.float32, device="cuda")
        f.spmm(dev(B2), Cd, tileK=64)
        torch.cuda.synchronize()
    R, L1 = orc.spmm_csr(A.row_ptr, A.col, A.val, A.M, B, mode=0)
    ok, worst, row = row_l1_parity(Cd.cpu().numpy(), R, L1, 1e-5)
    assert ok, (worst, row)


def test_rcm_limits_give_up_cleanly():
    """The ordering's loops run to proven maxima (N + 1 levels, N (ceil(lg N) + 2) + 1
    component rounds) that a correct walk never reaches.  Lowered from the host, they make the
    walk stop -- inside the work-group kernel, which then ends normally, or between the
    host-driven levels -- and the call returns ERR_STATE; restored, the same call succeeds."""
    rp, col = banded(2000, 1)  # a path: 1999 levels
    L = vm.lib()
    try:
        for levels, rounds, what in ((50, 0, b"levels"), (0, 1, b"rounds")):
            assert L.vcsrmc_set_rcm_limits(levels, rounds) == vm.OK
            say("rcm limits", levels, rounds)
            with pytest.raises(vm.VCSRMCError) as e:
                gpu_rcm(rp, col, 2000, 2000)
            assert e.value.status == vm.ERR_STATE and what.decode() in str(e.value)
        A = vm.generate(2, 30000)  # frontiers beyond one work-group: host-driven levels
        assert L.vcsrmc_set_rcm_limits(2, 0) == vm.OK
        say("rcm limits host levels", A.N)
        with pytest.raises(vm.VCSRMCError) as e:
            gpu_rcm(A.row_ptr, A.col, A.M, A.N)
        assert e.value.status == vm.ERR_STATE
    finally:
        assert L.vcsrmc_set_rcm_limits(0, 0) == vm.OK
    assert np.array_equal(gpu_rcm(rp, col, 2000, 2000), 1999 - np.arange(2000))


def test_apply_duplicate_leaves_csr_unchanged():
    """A row holding one column twice is refused before anything is written."""
    rp = np.array([0, 1, 3], np.int32)
    col, val = np.array([2, 0, 0], np.int32), np.array([1.5, 2.5, 3.5], np.float32)
    dc, dv = dev(col), dev(val)
    with pytest.raises(vm.VCSRMCError) as e:
        vm.apply_column_permutation_device(dev(rp), dc, dv, 2, 3,
                                           dev(np.array([2, 1, 0], np.int32)))
    assert e.value.status == vm.ERR_UNSORTED
    assert np.array_equal(dc.cpu().numpy(), col) and np.array_equal(dv.cpu().numpy(), val)
