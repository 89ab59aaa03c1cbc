"""Writes tests/golden/vcsrmc_golden.npz: small seeded CSR inputs and the VCSRMC arrays that the
reference's own csr_to_vcsr_mc (MuuSeoTia/VCSR_MC src/vcsr_mc.cu:25-123, compiled from its
sources by oracle/Makefile into oracle/_ref) returns for them, in the reference's own tie order.

Run from the repository root:  python tests/golden/make_golden.py
Needs oracle/_ref (built only where the reference sources are present).
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
import vcsr_mc_amd as vm  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "vcsrmc_golden.npz")


def rand_csr(rng, M, N, density=None, per_row=None, mag=1.0, empty_frac=0.0):
    rows = []
    for _ in range(M):
        if rng.random() < empty_frac:
            k = 0
        elif per_row is not None:
            k = min(N, int(rng.poisson(per_row)))
        else:
            k = int(rng.binomial(N, density))
        rows.append(np.sort(rng.choice(N, size=k, replace=False)))
    rp = np.zeros(M + 1, np.int32)
    rp[1:] = np.cumsum([len(r) for r in rows])
    col = np.concatenate(rows).astype(np.int32) if rp[-1] else np.zeros(0, np.int32)
    val = (rng.uniform(-1, 1, col.size) * mag).astype(np.float32)
    return rp, col, val


def cases():
    rng = np.random.default_rng(20260923)
    out = []
    n = 50
    out.append(("diagonal", np.arange(n + 1, dtype=np.int32), np.arange(n, dtype=np.int32),
                rng.uniform(-1, 1, n).astype(np.float32), n, n, 16, False))
    for segw in (16, 32, 48, 64):
        for fp32 in (False, True):
            rp, c, v = rand_csr(rng, 37, 45 + segw, density=0.15)
            out.append((f"random_s{segw}_{'fp32' if fp32 else 'fp16'}", rp, c, v, 37, 45 + segw,
                        segw, fp32))
    # two block rows of dense 32x32 blocks at block columns {0, 2} and {1, 2}
    rows = []
    for r in range(64):
        bcs = (0, 2) if r < 32 else (1, 2)
        rows.append(np.concatenate([np.arange(32 * b, 32 * b + 32) for b in bcs]))
    rp = np.zeros(65, np.int32)
    rp[1:] = np.cumsum([len(x) for x in rows])
    col = np.concatenate(rows).astype(np.int32)
    out.append(("dense_blocks", rp, col, rng.normal(size=col.size).astype(np.float32), 64, 96,
                32, False))
    rp, c, v = rand_csr(rng, 40, 70, density=0.08, empty_frac=0.3)
    out.append(("empty_rows_ragged_N", rp, c, v, 40, 70, 32, False))
    out.append(("nnz0", np.zeros(6, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32),
                5, 7, 16, False))
    rp, c, v = rand_csr(rng, 30, 60, density=0.2, mag=1e5)
    out.append(("scale_large", rp, c, v, 30, 60, 16, False))
    rp, c, v = rand_csr(rng, 30, 60, density=0.2, mag=4e-5)
    out.append(("scale_tiny", rp, c, v, 30, 60, 32, False))
    for cfg, size, segw, fp32 in ((2, 400, 32, False), (3, 6, 32, True), (4, 6, 32, False),
                                  (5, 9, 32, False), (1, 300, 32, True)):
        A = vm.generate(cfg, size)
        out.append((f"workload{cfg}_size{size}", A.row_ptr, A.col, A.val, A.M, A.N, segw, fp32))
    return out


def main():
    oracle.build(ref=True)
    data, manifest = {}, []
    for i, (name, rp, c, v, M, N, segw, fp32) in enumerate(cases()):
        f = oracle.ref_build_format(rp, c, v, M, N, segw, fp32)
        key = f"c{i}"
        data[f"{key}/row_ptr"] = np.asarray(rp, np.int32)
        data[f"{key}/col"] = np.asarray(c, np.int32)
        data[f"{key}/val"] = np.asarray(v, np.float32)
        for a in oracle.ARRAYS:
            data[f"{key}/ref_{a}"] = f[a]
        manifest.append(dict(key=key, name=name, M=int(M), N=int(N), segw=int(segw),
                             fp32=bool(fp32), scale=float(f["scale"]),
                             scale_bits=int(np.float32(f["scale"]).view(np.uint32)),
                             num_segments=int(f["num_segments"]), G=int(len(f["group_depth"])),
                             nitems=int(len(f["item_gbeg"]))))
        print(name, "G", len(f["group_depth"]), "nval", len(f["val"]), "items",
              len(f["item_gbeg"]), "scale", f["scale"])
    data["manifest"] = np.frombuffer(json.dumps(manifest).encode(), dtype=np.uint8)
    np.savez_compressed(OUT, **data)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
