"""Writes tests/golden/rcm_golden.npz: small CSR inputs with the positions that the reference's
own rcm_column_order returns for them, the CSR and B that its apply_column_permutation makes
(MuuSeoTia/VCSR_MC include/reorder.hpp:17-108, compiled from the header where it lies by
oracle/Makefile into oracle/_ref), and std::sort results for tie-heavy and adversarial inputs
(the call the reference makes at reorder.hpp:67-68, as compiled here).

Run from the repository root:  python tests/golden/make_rcm_golden.py
Needs oracle/_ref (built only where the reference sources are present).
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

sys.path.insert(0, os.path.join(ROOT, "tests"))
from golden_io import adversary_hub  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "rcm_golden.npz")


def csr_from_rows(rows, M):
    rp = np.zeros(M + 1, np.int32)
    rp[1:] = np.cumsum([len(r) for r in rows])
    col = np.concatenate([np.asarray(r, np.int64) for r in rows]).astype(np.int32) if rp[-1] \
        else np.zeros(0, np.int32)
    return rp, col


def rand_rows(rng, M, N, per_row, skew):
    rows = []
    for _ in range(M):
        k = min(N, int(rng.poisson(per_row)))
        if skew:
            c = np.unique((N * rng.random(k) ** 3).astype(np.int64))
        else:
            c = np.sort(rng.choice(N, size=k, replace=False))
        rows.append(c)
    return rows


def cases():
    rng = np.random.default_rng(20260923)
    out = []
    # star: column 0 joined to 1..40 (the children of 0 tie on degree 1: introsort order)
    k = 40
    rows = [np.arange(1, k + 1)] + [[0] for _ in range(k)]
    out.append(("star41",) + csr_from_rows(rows, k + 1) + (k + 1, k + 1))
    # two stars and isolated columns, M < N
    rows = [np.arange(1, 25), [0], [0], [30], np.arange(31, 60)]
    out.append(("stars_isolated",) + csr_from_rows(rows, 5) + (5, 70))
    # more rows than columns: rows >= N only add self-loops
    rows = [[1, 2], [0], [3], [2], [0, 3], [1], [2, 3]]
    out.append(("tall",) + csr_from_rows(rows, 7) + (7, 4))
    for i, (M, N, d, skew) in enumerate([(60, 60, 3, False), (200, 150, 6, True),
                                         (500, 500, 10, True), (300, 800, 4, True),
                                         (900, 400, 2, False), (1000, 1000, 8, True)]):
        out.append((f"random{i}",) + csr_from_rows(rand_rows(rng, M, N, d, skew), M) + (M, N))
    return out


def adversary_star(keys):
    """Vertex 0 is a leaf of hub 1; hub 1's children are 2 .. n+1, child 2+i with keys[i]
    private leaves, so its degree is keys[i] + 1.  The BFS starts at leaf 0 (the lowest id of
    degree 1), reaches the hub, and sorts the hub's children by degree: the comparisons of an
    adversarial std::sort input, which end in the heapsort fallback."""
    n = len(keys)
    N = 2 + n + int(np.sum(keys))
    adj = [[] for _ in range(N)]

    def edge(u, v):
        adj[u].append(v)
        adj[v].append(u)
    edge(0, 1)
    nxt = 2 + n
    for i, k in enumerate(keys):
        edge(1, 2 + i)
        for _ in range(int(k)):
            edge(2 + i, nxt)
            nxt += 1
    rp, col = csr_from_rows([sorted(a) for a in adj], N)
    return rp, col, N


def main():
    oracle.build(ref=True)
    if not oracle.ref_available():
        sys.exit("oracle/_ref is not built (the reference sources are needed)")
    rng = np.random.default_rng(7)
    data = {}
    names = []
    all_cases = cases()
    rp, col, N = adversary_star(oracle.ref_sort_adversary(200) // 2)
    all_cases.append(("adversary_star200", rp, col, N, N))
    for name, rp, col, M, N in all_cases:
        pos = oracle.ref_rcm_order(rp, col, M, N)
        val = rng.uniform(-1, 1, col.size).astype(np.float32)
        O = 3 if N <= 2000 else 1
        B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
        c2, v2, B2 = oracle.ref_apply_column_permutation(rp, col, val, M, N, pos, B.reshape(-1), O)
        data.update({f"{name}/row_ptr": rp, f"{name}/col": col, f"{name}/val": val,
                     f"{name}/shape": np.array([M, N], np.int32), f"{name}/position": pos,
                     f"{name}/B": B, f"{name}/new_col": c2, f"{name}/new_val": v2,
                     f"{name}/new_B": B2.reshape(N, O)})
        names.append(name)
    sorts = []
    for i, (n, nk) in enumerate([(17, 1), (40, 1), (100, 2), (257, 3), (1000, 5), (1000, 1),
                                 (3000, 40)]):
        key = rng.integers(0, nk, size=n + 10).astype(np.int32)
        a = rng.permutation(n + 10)[:n].astype(np.int32)
        data[f"sort{i}/a"] = a
        data[f"sort{i}/key"] = key
        data[f"sort{i}/sorted"] = oracle.ref_std_sort_by_key(a, key)
        sorts.append(f"sort{i}")
    # adversarial keys (McIlroy) drive std::sort into its heapsort fallback; halving them makes
    # pairs of equal keys while the fallback is still reached
    for n in (200, 1000, 5000):
        key = oracle.ref_sort_adversary(n) // 2
        a = np.arange(n, dtype=np.int32)
        name = f"adversary{n}"
        data[f"{name}/a"] = a
        data[f"{name}/key"] = key.astype(np.int32)
        data[f"{name}/sorted"] = oracle.ref_std_sort_by_key(a, key)
        sorts.append(name)
    # a 2000-child hub whose degrees are adversarial std::sort keys: the sort of that group is
    # partitioned by work-groups on the GPU and reaches the heapsort fallback on a large range
    keys = (oracle.ref_sort_adversary(2000) // 2).astype(np.int32)
    rp, col, N = adversary_hub(keys)
    data["hub2000/keys"] = keys
    data["hub2000/position"] = oracle.ref_rcm_order(rp, col, N, N)
    data["cases"] = np.array(names)
    data["sorts"] = np.array(sorts)
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT}: {len(names)} matrices, {len(sorts)} sorts")


if __name__ == "__main__":
    main()
