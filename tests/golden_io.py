"""Loader for tests/golden/vcsrmc_golden.npz (written by tests/golden/make_golden.py from the
reference's own csr_to_vcsr_mc), and builders of the structured patterns the reordering tests
share."""
import json
import os

import numpy as np

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "vcsrmc_golden.npz")
ARRAYS = ("group_ptr", "group_depth", "group_seg_base", "group_rows", "lcol", "val",
          "item_gbeg", "item_gend")


def load_cases():
    z = np.load(PATH, allow_pickle=False)
    manifest = json.loads(bytes(z["manifest"]).decode())
    out = []
    for m in manifest:
        k = m["key"]
        case = dict(m)
        case["row_ptr"] = z[f"{k}/row_ptr"]
        case["col"] = z[f"{k}/col"]
        case["val"] = z[f"{k}/val"]
        ref = dict(M=m["M"], N=m["N"], segw=m["segw"], bundle=16, num_segments=m["num_segments"],
                   scale=np.uint32(m["scale_bits"]).view(np.float32), fp32=m["fp32"])
        for a in ARRAYS:
            ref[a] = z[f"{k}/ref_{a}"]
        case["ref"] = ref
        out.append(case)
    return out


def adversary_hub(keys):
    """Symmetric pattern whose BFS sorts one large child group by the given degrees.

    Vertex 0 is a leaf of hub 1 and, with the lowest (degree, id), the BFS root; the hub's
    children are 2 .. n+1; child 2+i is joined to donors 0 .. keys[i]-1 of a shared pool
    (vertices n+2 ...), so its degree is keys[i] + 1 and the hub's children are sorted by keys.
    Returns (row_ptr, col, N)."""
    keys = np.asarray(keys, np.int64)
    n = len(keys)
    donors = int(keys.max()) if n else 0
    N = 2 + n + donors
    src = [np.array([0, 1]), np.full(n, 1), 2 + np.arange(n)]
    dst = [np.array([1, 0]), 2 + np.arange(n), np.full(n, 1)]
    child = np.repeat(2 + np.arange(n), keys)
    donor = 2 + n + (np.arange(int(keys.sum())) - np.repeat(np.cumsum(keys) - keys, keys))
    src += [child, donor]
    dst += [donor, child]
    r = np.concatenate(src)
    c = np.concatenate(dst)
    order = np.lexsort((c, r))
    r, c = r[order], c[order]
    rp = np.zeros(N + 1, np.int64)
    np.add.at(rp, r + 1, 1)
    return np.cumsum(rp).astype(np.int32), c.astype(np.int32), N


def banded(N, bw):
    """N x N pattern with columns r - bw .. r + bw in row r."""
    r = np.repeat(np.arange(N), 2 * bw + 1)
    c = r + np.tile(np.arange(-bw, bw + 1), N)
    keep = (c >= 0) & (c < N)
    rp = np.zeros(N + 1, np.int64)
    np.add.at(rp, r[keep] + 1, 1)
    return np.cumsum(rp).astype(np.int32), c[keep].astype(np.int32)


def grid5(nx, ny):
    """5-point stencil on an nx x ny grid, vertex x * ny + y."""
    rows = []
    for x in range(nx):
        for y in range(ny):
            v = x * ny + y
            rows.append(sorted(w for w, ok in ((v - ny, x > 0), (v - 1, y > 0), (v, True),
                                               (v + 1, y < ny - 1), (v + ny, x < nx - 1)) if ok))
    rp = np.zeros(len(rows) + 1, np.int32)
    rp[1:] = np.cumsum([len(r) for r in rows])
    return rp, np.concatenate(rows).astype(np.int32)


def csr_from_edges(M, N, edges):
    """CSR pattern (values 1) of the (row, column) pairs that fall inside M x N, duplicates
    merged."""
    rows = [[] for _ in range(M)]
    for r, c in edges:
        if 0 <= r < M and 0 <= c < N:
            rows[r].append(c)
    rows = [np.unique(np.asarray(x, np.int64)) for x in rows]
    rp = np.zeros(M + 1, np.int32)
    rp[1:] = np.cumsum([len(x) for x in rows])
    col = np.concatenate(rows).astype(np.int32) if rp[-1] else np.zeros(0, np.int32)
    return rp, col
