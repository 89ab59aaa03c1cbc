"""Handles on several host threads at once.  A handle holds all of its format's state; what the
library shares between handles is read-only or synchronised (the row-grouping mode and the RCM
limits are atomics, the per-device scratch lookup takes a mutex).  So four threads that each
build their own format and multiply on their own stream, at the same time, must produce bit for
bit what the same calls produce one after another on one thread.  The matrices have no split
panels, so every product is deterministic (no atomics)."""
import threading

import numpy as np
import pytest

import vcsr_mc_amd as vm
from conftest import random_csr
from gpu_util import row_l1_parity, say

pytestmark = pytest.mark.gpu

TAU = {True: 1e-5, False: 2e-3}


def _cases():
    out = []
    for i in range(4):
        rng = np.random.default_rng(4100 + i)
        M, N = 2500 + 700 * i, 2000 + 300 * i
        rp, c, v = random_csr(rng, M, N, nnz_per_row=5 + 2 * i, empty_frac=0.1 * i)
        fp32 = bool(i % 2)
        O = 40 + 32 * i
        B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
        if not fp32:
            B = B.astype(np.float16).astype(np.float32)
        C0 = rng.uniform(-1, 1, (M, O)).astype(np.float32)
        out.append(dict(rp=rp, c=c, v=v, M=M, N=N, fp32=fp32, B=B, C0=C0))
    return out


def _run(case, stream):
    """Build, then C += A.B and C = A.B twice each on `stream`; returns the four results."""
    import torch
    with torch.cuda.stream(stream):
        d = {k: torch.from_numpy(case[k]).to("cuda", non_blocking=False)
             for k in ("rp", "c", "v", "B", "C0")}
        outs = []
        with vm.DeviceFormat.from_device_csr(d["rp"], d["c"], d["v"], case["M"], case["N"],
                                             case["fp32"], 32, stream=stream) as f:
            info = f.info()
            for overwrite in (False, False, True, True):
                C = d["C0"].clone()
                f.spmm(d["B"], C, tileK=128, overwrite=overwrite, stream=stream)
                outs.append(C)
        stream.synchronize()
        return info, [C.cpu().numpy() for C in outs]


def test_handles_on_threads(orc):
    import torch
    cases = _cases()
    say("threads: serial")
    serial = [_run(case, torch.cuda.Stream()) for case in cases]
    for (info, outs), case in zip(serial, cases):
        assert info["num_split_panels"] == 0, info
        R, L1 = orc.spmm_csr(case["rp"], case["c"], case["v"], case["M"], case["B"],
                             mode=0 if case["fp32"] else 1, scale=info["scale"])
        touched = np.diff(case["rp"]) > 0
        for k, got in enumerate(outs):
            base = case["C0"].astype(np.float64).copy()
            if k >= 2:
                base[touched] = 0.0
            ok, worst, row = row_l1_parity(got, R + base, L1 + np.abs(base).sum(axis=1),
                                           TAU[case["fp32"]])
            assert ok, f"serial call {k}: row {row}: error / bound = {worst:.3g}"
    for rep in range(3):
        say("threads: concurrent", rep)
        results = [None] * len(cases)
        errors = []
        start = threading.Barrier(len(cases))

        def worker(i):
            try:
                stream = torch.cuda.Stream()
                start.wait(timeout=60)
                results[i] = _run(cases[i], stream)
            except BaseException as e:  # reported on the main thread
                errors.append((i, repr(e)))

        threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(cases))]
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=120)
        assert not any(t.is_alive() for t in threads), "a worker did not finish"
        assert not errors, errors
        for i, ((info_s, outs_s), (info_c, outs_c)) in enumerate(zip(serial, results)):
            assert info_s == info_c, i
            for k, (a, b) in enumerate(zip(outs_s, outs_c)):
                assert np.array_equal(a, b), (rep, i, k)
