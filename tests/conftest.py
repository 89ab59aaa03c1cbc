import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.build()
    return oracle


def random_csr(rng, M, N, density=None, nnz_per_row=None, heavy_rows=0, heavy_nnz=0,
               mag=1.0, empty_frac=0.0):
    """Random CSR with sorted, distinct columns per row (host numpy arrays)."""
    rows = []
    for r in range(M):
        if rng.random() < empty_frac:
            k = 0
        elif nnz_per_row is not None:
            k = min(N, int(rng.poisson(nnz_per_row)))
        else:
            k = int(rng.binomial(N, density))
        rows.append(np.sort(rng.choice(N, size=k, replace=False)) if k else np.zeros(0, np.int64))
    for r in rng.choice(M, size=min(heavy_rows, M), replace=False) if heavy_rows else []:
        k = min(N, heavy_nnz)
        rows[r] = np.sort(rng.choice(N, size=k, replace=False))
    rp = np.zeros(M + 1, np.int32)
    rp[1:] = np.cumsum([len(c) for c in rows])
    col = np.concatenate(rows).astype(np.int32) if rp[-1] else np.zeros(0, np.int32)
    val = (rng.uniform(-1, 1, size=col.size) * mag).astype(np.float32)
    return rp, col, val


@pytest.fixture
def rng():
    return np.random.default_rng(20260923)
