"""The oracle's column reordering (oracle/rcm_oracle.c) pinned against the reference's
rcm_column_order / apply_column_permutation (include/reorder.hpp:17-108) and std::sort:
committed fixtures made by the reference's compiled header (tests/golden/make_rcm_golden.py),
the compiled header itself where oracle/_ref is built, and closed forms."""
import os

import numpy as np
import pytest

from conftest import random_csr

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "rcm_golden.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN)


def csr_from_rows(rows, M):
    rp = np.zeros(M + 1, np.int32)
    rp[1:] = np.cumsum([len(r) for r in rows])
    col = np.concatenate([np.asarray(r, np.int64) for r in rows]).astype(np.int32) if rp[-1] \
        else np.zeros(0, np.int32)
    return rp, col


def test_std_sort_fixtures(orc, gold):
    for s in gold["sorts"]:
        got = orc.std_sort_by_key(gold[f"{s}/a"], gold[f"{s}/key"])
        assert np.array_equal(got, gold[f"{s}/sorted"]), s


def test_std_sort_closed_forms(orc):
    rng = np.random.default_rng(1)
    for n in range(0, 70):
        key = rng.integers(0, 4, size=n).astype(np.int32)
        a = np.arange(n, dtype=np.int32)
        got = orc.std_sort_by_key(a, key)
        assert sorted(got.tolist()) == list(range(n))
        assert np.all(np.diff(key[got]) >= 0)
        if n <= 16:  # insertion sort only: stable
            assert np.array_equal(got, np.argsort(key, kind="stable"))
    # all keys equal, 17+ elements: the partitions reorder equal elements (not stable)
    got = orc.std_sort_by_key(np.arange(40, dtype=np.int32), np.zeros(40, np.int32))
    assert not np.array_equal(got, np.arange(40))


def test_std_sort_against_compiled(orc):
    if not orc.ref_available():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    rng = np.random.default_rng(2)
    for t in range(400):
        n = int(rng.integers(0, 600))
        key = rng.integers(0, int(rng.integers(1, 8)), size=n + 5).astype(np.int32)
        a = rng.permutation(n + 5)[:n].astype(np.int32)
        assert np.array_equal(orc.std_sort_by_key(a, key), orc.ref_std_sort_by_key(a, key)), t


def test_heap_sort_step(orc):
    rng = np.random.default_rng(5)
    for n in range(0, 40):
        key = rng.integers(0, 3, size=n).astype(np.int32)
        got = orc.heap_sort_by_key(np.arange(n, dtype=np.int32), key)
        assert sorted(got.tolist()) == list(range(n)) and np.all(np.diff(key[got]) >= 0)
    if not orc.ref_available():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    for t in range(300):
        n = int(rng.integers(0, 500))
        key = rng.integers(0, int(rng.integers(1, 6)), size=n + 3).astype(np.int32)
        a = rng.permutation(n + 3)[:n].astype(np.int32)
        assert np.array_equal(orc.heap_sort_by_key(a, key), orc.ref_partial_sort_by_key(a, key))


def test_rcm_fixtures(orc, gold):
    for name in gold["cases"]:
        rp, col = gold[f"{name}/row_ptr"], gold[f"{name}/col"]
        M, N = (int(x) for x in gold[f"{name}/shape"])
        pos = orc.rcm_order(rp, col, M, N)
        assert np.array_equal(pos, gold[f"{name}/position"]), name
        c2, v2, B2 = orc.apply_column_permutation(rp, col, gold[f"{name}/val"], M, N, pos,
                                                  gold[f"{name}/B"], gold[f"{name}/B"].shape[1])
        assert np.array_equal(c2, gold[f"{name}/new_col"]), name
        assert np.array_equal(v2, gold[f"{name}/new_val"]), name
        assert np.array_equal(B2, gold[f"{name}/new_B"]), name


def test_rcm_adversarial_hub(orc, gold):
    from golden_io import adversary_hub
    rp, col, N = adversary_hub(gold["hub2000/keys"])
    assert np.array_equal(orc.rcm_order(rp, col, N, N), gold["hub2000/position"])


def test_rcm_against_compiled(orc):
    if not orc.ref_available():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    rng = np.random.default_rng(3)
    for t in range(60):
        M, N = int(rng.integers(1, 300)), int(rng.integers(1, 300))
        rp, col, _ = random_csr(rng, M, N, nnz_per_row=float(rng.uniform(0, 8)),
                                heavy_rows=int(rng.integers(0, 3)), heavy_nnz=60)
        assert np.array_equal(orc.rcm_order(rp, col, M, N), orc.ref_rcm_order(rp, col, M, N)), t


def test_rcm_band_and_grid_against_compiled(orc):
    """Structured patterns (deep walks, wide anti-diagonal levels) beside the random ones."""
    if not orc.ref_available():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    from golden_io import banded, grid5
    for rp, col in (banded(3000, 1), banded(2500, 4), grid5(40, 70), grid5(1, 300)):
        N = rp.size - 1
        assert np.array_equal(orc.rcm_order(rp, col, N, N), orc.ref_rcm_order(rp, col, N, N))


def test_rcm_path_graph(orc):
    # tridiagonal: vertex 0 has the lowest (degree, id), the BFS walks 0, 1, ..., N-1
    N = 50
    rows = [[j for j in (i - 1, i, i + 1) if 0 <= j < N] for i in range(N)]
    rp, col = csr_from_rows(rows, N)
    assert np.array_equal(orc.rcm_order(rp, col, N, N), N - 1 - np.arange(N))


def test_rcm_star_and_isolated(orc):
    # star 0 - {1..k}, k <= 17: leaf 1 is the root, then 0, then leaves 2..k in ascending id
    # (the children list of 0 has k - 1 <= 16 entries: insertion sort keeps id order).
    # Columns k+1 .. k+3 are isolated (degree 0) and come first, in id order.
    k = 12
    N = k + 4
    rows = [np.arange(1, k + 1)] + [[0] for _ in range(k)]
    rp, col = csr_from_rows(rows, k + 1)
    order = [k + 1, k + 2, k + 3, 1, 0] + list(range(2, k + 1))
    expect = np.empty(N, np.int32)
    expect[np.array(order)] = N - 1 - np.arange(N)
    assert np.array_equal(orc.rcm_order(rp, col, k + 1, N), expect)


def test_rcm_rows_beyond_n_add_self_loops(orc):
    # Star 0 - {1, 2, 3} (rows 0..3, N = 4) plus row 4 >= N holding column 2: that row only
    # gives column 2 a self-loop, so its degree is 2 against 1 for leaves 1 and 3.  Leaf 1 is
    # the root, then 0; the children of 0 sorted by degree are 3 (degree 1) before 2.
    rows = [[1, 2, 3], [0], [0], [0], [2]]
    rp, col = csr_from_rows(rows, 5)
    assert np.array_equal(orc.rcm_order(rp, col, 5, 4), np.array([2, 3, 0, 1]))  # 1, 0, 3, 2
    # without row 4 the children keep id order: 1, 0, 2, 3
    assert np.array_equal(orc.rcm_order(rp[:5], col[:rp[4]], 4, 4), np.array([2, 3, 1, 0]))


def test_apply_is_a_relabelling(orc):
    rng = np.random.default_rng(4)
    M, N, O = 80, 120, 5
    rp, col, val = random_csr(rng, M, N, nnz_per_row=6)
    pos = orc.rcm_order(rp, col, M, N)
    assert sorted(pos.tolist()) == list(range(N))
    B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
    c2, v2, B2 = orc.apply_column_permutation(rp, col, val, M, N, pos, B, O)
    for r in range(M):
        s, e = rp[r], rp[r + 1]
        assert np.all(np.diff(c2[s:e]) > 0)
        assert dict(zip(pos[col[s:e]].tolist(), val[s:e].tolist())) == \
            dict(zip(c2[s:e].tolist(), v2[s:e].tolist()))
    assert np.array_equal(B2[pos], B)
    # C = (A P)(P^T B) = A B, the products summed in another order
    R1 = np.zeros((M, O)); R2 = np.zeros((M, O))
    orc.lib().orc_cpu_spmm_f64(*(orc._p(x, t) for x, t in ((rp, orc.C.c_int), (col, orc.C.c_int),
                                                           (val, orc.C.c_float))), M,
                               orc._p(B, orc.C.c_float), O, orc._p(R1, orc.C.c_double))
    orc.lib().orc_cpu_spmm_f64(*(orc._p(x, t) for x, t in ((rp, orc.C.c_int), (c2, orc.C.c_int),
                                                           (v2, orc.C.c_float))), M,
                               orc._p(B2, orc.C.c_float), O, orc._p(R2, orc.C.c_double))
    assert np.allclose(R1, R2, rtol=0, atol=1e-12)
