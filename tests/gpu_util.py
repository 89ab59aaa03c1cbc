"""Helpers for the GPU parity tests: device copies, the parity norm, row sampling."""
import sys

import numpy as np


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def say(*args):
    """Names the case before a GPU step, flushed, so a failing run says where it was."""
    print("[case]", *args, flush=True)
    sys.stdout.flush()


def row_l1_parity(C_gpu, R, L1, tau):
    """Per row r: ||C_gpu[r] - R[r]||_1 <= tau * L1[r] (+ a denormal-scale floor).
    Returns (ok, worst ratio, worst row)."""
    C = np.asarray(C_gpu, np.float64)
    err = np.abs(C - R).sum(axis=1)
    bound = tau * L1 + 1e-30
    ratio = err / bound
    worst = int(np.argmax(ratio)) if ratio.size else -1
    return bool(np.all(err <= bound)), float(ratio.max()) if ratio.size else 0.0, worst


def sub_csr(rp, c, v, rows):
    """CSR of the given rows only (same columns)."""
    rows = np.asarray(rows)
    lens = rp[rows + 1] - rp[rows]
    out_rp = np.zeros(len(rows) + 1, np.int32)
    out_rp[1:] = np.cumsum(lens)
    idx = np.concatenate([np.arange(rp[r], rp[r + 1]) for r in rows]) if out_rp[-1] else \
        np.zeros(0, np.int64)
    return out_rp, c[idx].astype(np.int32), v[idx].astype(np.float32)
