"""Loader for tests/golden/vcsrmc_golden.npz (written by tests/golden/make_golden.py from the
reference's own csr_to_vcsr_mc)."""
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
