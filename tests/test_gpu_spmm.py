"""GPU SpMM vs the oracle.  Parity gate: per row r,
    ||C_gpu[r,:] - C_ref[r,:]||_1 <= tau * sum_k sum_p |a_rp b_{c_p,k}|,
tau = 1e-5 for FP32 inputs and 2e-3 for FP16 inputs, with C_ref the oracle's double-precision
product of the same (FP16-quantised, for vcsr_mc) operands.  Where C starts non-zero the norm
also counts what is already in the row, + ||C0[r,:]||_1 (C += A.B rounds the final sum)."""
import numpy as np
import pytest

import vcsr_mc_amd as vm
from conftest import random_csr
from gpu_util import dev, row_l1_parity, say, sub_csr

pytestmark = pytest.mark.gpu

TAU = {True: 1e-5, False: 2e-3}


def run_spmm(rp, c, v, M, N, B, fp32, tileK=128, segw=32, b16=False, C0=None, upload=None):
    import torch
    if upload is None:
        f = vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, N, fp32, segw)
    else:
        f = vm.DeviceFormat.from_host_format(upload)
    with f:
        dB = dev(B)
        if b16:
            dB = dB.half()
        C = dev(C0) if C0 is not None else torch.zeros((M, B.shape[1]), dtype=torch.float32,
                                                       device="cuda")
        f.spmm(dB, C, tileK=tileK)
        torch.cuda.synchronize()
        return C.cpu().numpy(), f.info()


def check(orc, rp, c, v, M, N, B, fp32, **kw):
    C, info = run_spmm(rp, c, v, M, N, B, fp32, **kw)
    scale = info["scale"]
    R, L1 = orc.spmm_csr(rp, c, v, M, B, mode=0 if fp32 else 1, scale=scale)
    if kw.get("C0") is not None:
        R = R + kw["C0"].astype(np.float64)
    ok, worst, row = row_l1_parity(C, R, L1, TAU[fp32])
    assert ok, f"row {row}: error / bound = {worst:.3g}"
    return C, R


@pytest.mark.parametrize("fp32", [False, True])
@pytest.mark.parametrize("tileK", [16, 32, 64, 128])
def test_random_all_tiles(orc, fp32, tileK):
    rng = np.random.default_rng(tileK + fp32)
    for O in (1, 7, 16, 100, 128, 256):
        M, N = int(rng.integers(1, 700)), int(rng.integers(1, 700))
        rp, c, v = random_csr(rng, M, N, density=float(rng.choice([0.002, 0.02, 0.2])),
                              empty_frac=0.2)
        B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
        say("random", fp32, tileK, O, M, N, c.size)
        check(orc, rp, c, v, M, N, B, fp32, tileK=tileK)


@pytest.mark.parametrize("fp32", [False, True])
def test_split_panels_and_accumulate(orc, fp32):
    """Heavy rows make panels of > 16 tiles (split units, atomic merge); C starts non-zero and
    rows A does not touch must come back bit-identical."""
    rng = np.random.default_rng(11)
    M, N, O = 900, 5000, 128
    rp, c, v = random_csr(rng, M, N, density=0.001, heavy_rows=5, heavy_nnz=4000,
                          empty_frac=0.3)
    B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, O)).astype(np.float32)
    C0[5] = -0.0
    say("split+accumulate", fp32)
    C, _ = check(orc, rp, c, v, M, N, B, fp32, C0=C0)
    empty = np.diff(rp) == 0
    assert C[empty].tobytes() == C0[empty].tobytes()


@pytest.mark.parametrize("M,N,kw", [(300, 400, dict(density=0.004)),
                                     (300, 400, dict(density=0.03)),
                                     (30000, 30000, dict(nnz_per_row=16))])
def test_fp16_b_matches_fp32_b(orc, M, N, kw):
    """FP16 B in HBM (converted by the caller) gives the same result as FP32 B, which the
    library rounds to binary16 either in the kernel (the two small cases) or in one conversion
    pass before it (B of 30,000 x 128 floats > 12 MB, tiles of fewer than 48 nonzeros,
    nnz >= 12 N); B itself is left untouched."""
    import torch
    rng = np.random.default_rng(12)
    rp, c, v = random_csr(rng, M, N, **kw)
    B = rng.uniform(-2, 2, (N, 128)).astype(np.float32)
    say("fp16 B vs fp32 B", M, N, len(c))
    with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, N, False, 32) as f:
        info = f.info()
        assert info["num_units"] == info["num_panels"]  # no split panel: no atomics
        converts = (len(c) >= 12 * N and len(c) < 48 * info["num_chunks"]
                    and N * 128 * 4 > 12 << 20)
        assert converts == (M == 30000)
        dB = dev(B)
        C1 = torch.zeros((M, 128), dtype=torch.float32, device="cuda")
        C2 = torch.zeros_like(C1)
        f.spmm(dB, C1, tileK=128)
        f.spmm(dB.half(), C2, tileK=128)
        torch.cuda.synchronize()
        assert np.array_equal(dB.cpu().numpy(), B)
        assert np.array_equal(C1.cpu().numpy(), C2.cpu().numpy())
    check(orc, rp, c, v, M, N, B, False)
    check(orc, rp, c, v, M, N, B, False, b16=True)


@pytest.mark.parametrize("O,tileK", [(128, 128), (256, 128), (192, 64), (128, 32), (160, 128)])
def test_converted_b_o_tile_major(orc, O, tileK):
    """An FP16 format given FP32 B above the conversion threshold rounds B to binary16 in one
    pass per call, laid out O-tile-major where the launch has several O tiles, all full (O tiles
    of 64 here for 128, 256 and 192 columns, of 32 at tileK 32) and row-major otherwise (160
    columns, O tiles of 64): the result equals the launch on the same B rounded by the caller,
    bit for bit, in both launch modes, and meets the parity norm."""
    import torch
    rng = np.random.default_rng(O + tileK)
    M = 30000
    rp, c, v = random_csr(rng, M, M, nnz_per_row=16)
    B = rng.uniform(-2, 2, (M, O)).astype(np.float32)
    say("converted B, O-tile-major", O, tileK, len(c))
    with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, M, False, 32) as f:
        info = f.info()
        assert info["num_units"] == info["num_panels"]  # no split panel: no atomics
        assert len(c) >= 12 * M and len(c) < 48 * info["num_chunks"] and M * O * 4 > 12 << 20
        tile = f.traffic_floor(O, tileK=tileK, b_f16=False)["o_tile_width"]
        assert (O % tile == 0 and O > tile) == (O != 160)
        dB = dev(B)
        for overwrite in (False, True):
            C1 = torch.full((M, O), 0.25, dtype=torch.float32, device="cuda")
            C2 = C1.clone()
            f.spmm(dB, C1, tileK=tileK, overwrite=overwrite)
            f.spmm(dB.half(), C2, tileK=tileK, overwrite=overwrite)
            torch.cuda.synchronize()
            assert torch.equal(C1, C2), overwrite
        assert np.array_equal(dB.cpu().numpy(), B)
    check(orc, rp, c, v, M, M, B, False, tileK=tileK)


@pytest.mark.parametrize("overwrite", [False, True])
def test_launcher_equals_spmm(overwrite):
    """The pre-bound launcher (checks and argument conversion once) enqueues the same launch as
    spmm: the same C bit for bit over repeated calls; a bad tileK is reported when called, and a
    call after the format is closed raises instead of passing the freed handle on."""
    import torch
    rng = np.random.default_rng(21)
    rp, c, v = random_csr(rng, 3000, 2500, density=0.01)
    B = dev(rng.uniform(-1, 1, (2500, 96)).astype(np.float32)).half()
    say("launcher", overwrite)
    with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), 3000, 2500, False, 32) as f:
        C1 = torch.full((3000, 96), 0.5, dtype=torch.float32, device="cuda")
        C2 = C1.clone()
        go = f.launcher(B, C2, tileK=64, overwrite=overwrite)
        for _ in range(3):
            f.spmm(B, C1, tileK=64, overwrite=overwrite)
            go()
        torch.cuda.synchronize()
        assert torch.equal(C1, C2)
        bad = f.launcher(B, C2, tileK=48)
        with pytest.raises(vm.VCSRMCError):
            bad()
    with pytest.raises(vm.VCSRMCError, match="closed"):
        go()


def test_scaled_values(orc):
    """|A| > 60000: A is divided by the range scale before FP16 and C multiplied back."""
    rng = np.random.default_rng(13)
    rp, c, v = random_csr(rng, 200, 300, density=0.05, mag=2e5)
    B = rng.uniform(-1, 1, (300, 64)).astype(np.float32)
    say("scaled")
    C, R = check(orc, rp, c, v, 200, 300, B, False)
    assert np.abs(R).max() > 1e4


def test_subnormal_fp16_values(orc):
    """Values that become binary16 subnormals must keep their value (no flush to zero)."""
    rng = np.random.default_rng(14)
    rp, c, v = random_csr(rng, 64, 64, density=0.3)
    v = (np.sign(v) * rng.uniform(1e-7, 6e-5, v.size)).astype(np.float32)
    v[0] = 1.0  # amax = 1: the range scale stays 1, small values stay subnormal
    B = rng.uniform(-1, 1, (64, 32)).astype(np.float32)
    say("subnormals")
    check(orc, rp, c, v, 64, 64, B, False)


@pytest.mark.parametrize("fp32", [False, True])
def test_upload_path_matches_build_path(orc, fp32):
    rng = np.random.default_rng(15)
    rp, c, v = random_csr(rng, 500, 500, density=0.02, heavy_rows=2, heavy_nnz=300)
    f = orc.build_format(rp, c, v, 500, 500, 16, fp32)
    V = vm.VCSRMC(M=500, N=500, segw=16, bundle=16, num_segments=f["num_segments"],
                  scale=float(f["scale"]), fp32=fp32, **{k: f[k] for k in vm._FMT_ARRAYS})
    B = rng.uniform(-1, 1, (500, 128)).astype(np.float32)
    say("upload path", fp32)
    C1, _ = run_spmm(rp, c, v, 500, 500, B, fp32, segw=16)
    C2, _ = run_spmm(rp, c, v, 500, 500, B, fp32, upload=V)
    _, L1 = orc.spmm_csr(rp, c, v, 500, B, mode=0 if fp32 else 1)
    ok, worst, _ = row_l1_parity(C1, C2.astype(np.float64), L1, 1e-6)
    assert ok, worst
    check(orc, rp, c, v, 500, 500, B, fp32, upload=V)


@pytest.mark.parametrize("fp32,row_steps,reach", [(False, 1, 16), (True, 0, 16), (True, 1, 4)])
def test_nonfinite_b_reach(fp32, row_steps, reach):
    """An Inf in B reaches exactly the rows multiplied together with its column: row 0 uses
    column 3 (Inf row); the other rows of its 16-row panel (tile steps) or of its 4-row group
    (FP32 row steps, the default for this matrix) do not (0 * Inf = NaN there); the rest of the
    panel, and row 17 in the next panel, never meet column 3 and stay finite; column 9's Inf
    row is used by no nonzero and reaches nothing."""
    import torch
    M, N, O = 40, 12, 32
    rows = {r: [5] for r in range(M)}
    rows[0] = [3, 5]
    rows[17] = [4, 5]
    rp = np.zeros(M + 1, np.int32)
    rp[1:] = np.cumsum([len(rows[r]) for r in range(M)])
    c = np.concatenate([rows[r] for r in range(M)]).astype(np.int32)
    v = np.full(c.size, 0.5, np.float32)
    B = np.ones((N, O), np.float32)
    B[3, :] = np.inf
    B[9, :] = np.inf
    say("non-finite B", fp32, row_steps)
    vm.set_fp32_row_steps(row_steps)
    try:
        with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, N, fp32, 32) as f:
            assert (f.info()["num_row_step_batches"] > 0) == (fp32 and row_steps == 1)
            Cd = torch.zeros((M, O), dtype=torch.float32, device="cuda")
            f.spmm(dev(B) if fp32 else dev(B).half(), Cd, tileK=32)
            torch.cuda.synchronize()
            C = Cd.cpu().numpy()
    finally:
        vm.set_fp32_row_steps(vm.FP32_ROW_STEPS_AUTO)
    assert np.all(np.isposinf(C[0]))
    assert np.all(np.isnan(C[1:reach]))
    expect = np.full((M - reach, O), 0.5, np.float32)
    expect[17 - reach] = 1.0  # row 17: columns 4 and 5
    assert np.array_equal(C[reach:], expect)


def test_empty_matrix():
    import torch
    say("empty")
    f = vm.DeviceFormat.from_device_csr(dev(np.zeros(6, np.int32)), dev(np.zeros(0, np.int32)),
                                        dev(np.zeros(0, np.float32)), 5, 7, False, 16)
    C = torch.full((5, 8), 3.0, device="cuda")
    B = torch.ones((7, 8), device="cuda")
    f.spmm(B, C)
    assert torch.all(C == 3.0)
    f.close()


def band_csr(rng, M, N, bw, mag):
    rows = [np.arange(max(0, min(r, N - 1) - bw), min(N, min(r, N - 1) + bw + 1)) for r in range(M)]
    rp = np.zeros(M + 1, np.int32)
    rp[1:] = np.cumsum([len(x) for x in rows])
    c = np.concatenate(rows).astype(np.int32)
    return rp, c, (rng.uniform(-1, 1, c.size) * mag).astype(np.float32)


@pytest.mark.parametrize("fp32", [False, True])
@pytest.mark.parametrize("tileK", [32, 128])
def test_mixed_tile_fill(orc, fp32, tileK):
    """One format holding nearly empty tiles, dense 16 x 32 blocks (dense copies) and three rows
    of 1500 nonzeros (a full row in every tile of their panels), with C starting non-zero and O
    past the last full O tile."""
    rng = np.random.default_rng(40 + tileK)
    M, N, O = 1000, 3000, 200
    rows = [np.sort(rng.choice(N, size=int(rng.poisson(3)), replace=False)) for _ in range(M)]
    for blk in range(0, M, 160):
        for r in range(blk, min(M, blk + 16)):
            rows[r] = np.union1d(rows[r], np.arange(64 + blk, 96 + blk))
    for r in (5, 333, 999):
        rows[r] = np.sort(rng.choice(N, size=1500, replace=False))
    rp = np.zeros(M + 1, np.int32)
    rp[1:] = np.cumsum([len(x) for x in rows])
    c = np.concatenate(rows).astype(np.int32)
    v = rng.uniform(-1, 1, c.size).astype(np.float32)
    B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, O)).astype(np.float32)
    say("mixed tile fill", fp32, tileK)
    check(orc, rp, c, v, M, N, B, fp32, tileK=tileK, C0=C0)


@pytest.mark.parametrize("tileK", [16, 32, 64, 128])
def test_fp32_entry_tiles(orc, tileK):
    """FP32 formats of more than 256 panels keep their sparse tiles as entry lists, scattered
    into the matrix-core operand through LDS: that path over 8,000-10,000-row matrices with
    about a quarter of the rows empty (moved after the others: at least ~6,000 rows, 375 panels,
    remain), two heavy rows (split panels) and sparse rows, O from 1 to 257, C starting
    non-zero."""
    rng = np.random.default_rng(900 + tileK)
    for O in (1, 7, 100, 128, 257):
        M, N = int(rng.integers(8000, 10000)), int(rng.integers(300, 9000))
        rp, c, v = random_csr(rng, M, N, nnz_per_row=float(rng.choice([3.0, 8.0])),
                              empty_frac=0.2, heavy_rows=2, heavy_nnz=3000)
        B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
        C0 = rng.uniform(-1, 1, (M, O)).astype(np.float32)
        say("fp32 entry tiles", tileK, O, M, N, c.size)
        C, info = run_spmm(rp, c, v, M, N, B, True, tileK=tileK, C0=C0)
        assert info["num_panels"] > 256 and info["num_dense"] < info["num_chunks"], info
        R, L1 = orc.spmm_csr(rp, c, v, M, B, mode=0, scale=info["scale"])
        R = R + C0.astype(np.float64)
        L1 = L1 + np.abs(C0.astype(np.float64)).sum(axis=1)
        ok, worst, r = row_l1_parity(C, R, L1, TAU[True])
        assert ok, f"row {r}: error / bound = {worst:.3g}"


def test_small_fp32_formats_all_dense():
    """An FP32 format of at most 256 panels and 4096 tiles stores every tile dense; the same
    matrix as an FP16 format, or one panel more, stores only tiles of more than 192 nonzeros."""
    rng = np.random.default_rng(77)
    for M, fp32, all_dense in ((4096, True, True), (4096, False, False), (4112, True, False)):
        rp, c, v = random_csr(rng, M, 4096, nnz_per_row=16)
        B = rng.uniform(-1, 1, (4096, 8)).astype(np.float32)
        _, info = run_spmm(rp, c, v, M, 4096, B, fp32)
        say("small fp32 all dense", M, fp32, info["num_panels"], info["num_chunks"],
            info["num_dense"])
        assert (info["num_dense"] == info["num_chunks"]) == all_dense, info


@pytest.mark.parametrize("keep", [1.0, 0.4])
@pytest.mark.parametrize("O", [100, 128])
def test_fp32_full_tiles_many_panels(orc, keep, O):
    """FP32 formats take O tiles of 128 only with at least 8192 panels and tiles of 48 or more
    nonzeros on average: a band of 49 diagonals over 8300 panels (keep = 1: dense tile copies;
    keep = 0.4: entry lists), O = 100 (B and C past the vector width) and 128, C starting
    non-zero, the whole product against the oracle."""
    rng = np.random.default_rng(int(O + 10 * keep))
    M = N = 8300 * 16
    rp, c, v = band_csr(rng, M, N, 24, 1.0)
    if keep < 1.0:
        row = np.repeat(np.arange(M), np.diff(rp))
        sel = rng.random(c.size) < keep
        rp = np.zeros(M + 1, np.int32)
        rp[1:] = np.cumsum(np.bincount(row[sel], minlength=M))
        c, v = c[sel], v[sel]
    B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, O)).astype(np.float32)
    say("fp32 full tiles, many panels", keep, O, c.size)
    C, info = run_spmm(rp, c, v, M, N, B, True, C0=C0)
    assert info["num_panels"] >= 8192 and info["nnz"] >= 48 * info["num_chunks"]
    R, L1 = orc.spmm_csr(rp, c, v, M, B, mode=0, scale=info["scale"])
    R = R + C0.astype(np.float64)
    L1 = L1 + np.abs(C0.astype(np.float64)).sum(axis=1)
    ok, worst, r = row_l1_parity(C, R, L1, TAU[True])
    assert ok, f"row {r}: error / bound = {worst:.3g}"


@pytest.mark.parametrize("seed", range(4))
def test_random_sweep(orc, seed):
    """Random shapes, patterns (uniform, Poisson rows with heavy rows, bands), value ranges,
    segw, tileK, O, FP16 / FP32 format and B, B and C base pointers off 16-byte alignment, and
    C0 = 0 or random: format arrays bit-exact and C = C0 + A.B within the parity norm.  With
    C0 != 0 the norm is that of everything summed into the row, sum |a||b| + ||C0[r]||_1: the
    final C0 + s rounds like any other addition (the reference's atomicAdd into C too), which a
    bound on sum |a||b| alone cannot cover when A's values are tiny."""
    import torch
    Os = [1, 3, 4, 7, 8, 16, 31, 33, 64, 65, 100, 127, 128, 129, 200, 256, 257]
    for t in range(12):
        rng = np.random.default_rng(7000 + 100 * seed + t)
        M, N = int(rng.integers(1, 2500)), int(rng.integers(1, 2500))
        kind = int(rng.integers(0, 3))
        mag = float(rng.choice([1.0, 1e5, 3e-5]))
        if kind == 0:
            rp, c, v = random_csr(rng, M, N, density=float(rng.choice([0.0005, 0.003, 0.03])),
                                  mag=mag, empty_frac=float(rng.uniform(0, 0.4)))
        elif kind == 1:
            rp, c, v = random_csr(rng, M, N, nnz_per_row=float(rng.uniform(0.5, 20)), mag=mag,
                                  heavy_rows=int(rng.integers(0, 5)),
                                  heavy_nnz=int(rng.integers(1, N + 1)))
        else:
            rp, c, v = band_csr(rng, M, N, int(rng.integers(0, 40)), mag)
        segw = int(rng.choice([16, 32, 48, 64]))
        fp32 = bool(rng.integers(0, 2))
        tileK = int(rng.choice([16, 32, 64, 128]))
        O = int(rng.choice(Os))
        b16 = (not fp32) and bool(rng.integers(0, 2))
        offB, offC = int(rng.random() < 0.3), int(rng.random() < 0.3)
        with_c0 = bool(rng.integers(0, 2))
        say("sweep", seed, t, M, N, c.size, kind, mag, segw, fp32, tileK, O, b16, offB, offC,
            with_c0)
        B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
        if not fp32:
            B = B.astype(np.float16).astype(np.float32)
        C0 = rng.uniform(-1, 1, (M, O)).astype(np.float32) if with_c0 else \
            np.zeros((M, O), np.float32)
        with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, N, fp32, segw) as f:
            scale = f.info()["scale"]
            V = f.download()
            got = {k: getattr(V, k) for k in ("M", "N", "segw", "bundle", "num_segments",
                                               "fp32", *vm._FMT_ARRAYS)}
            got["scale"] = np.float32(V.scale)
            assert orc.formats_equal(orc.Format(got),
                                     orc.build_format(rp, c, v, M, N, segw, fp32)) == [], t
            bt = torch.float16 if b16 else torch.float32
            dB = torch.empty(N * O + 8, dtype=bt, device="cuda")[offB:offB + N * O].view(N, O)
            dB.copy_(torch.from_numpy(B).to(bt))
            dC = torch.empty(M * O + 8, dtype=torch.float32, device="cuda")[offC:offC + M * O]
            dC = dC.view(M, O)
            dC.copy_(torch.from_numpy(C0))
            f.spmm(dB, dC, tileK=tileK)
            torch.cuda.synchronize()
            Cg = dC.cpu().numpy()
        R, L1 = orc.spmm_csr(rp, c, v, M, B, mode=0 if fp32 else 1, scale=scale)
        R = R + C0.astype(np.float64)
        L1 = L1 + np.abs(C0.astype(np.float64)).sum(axis=1)
        ok, worst, row = row_l1_parity(Cg, R, L1, TAU[fp32])
        assert ok, f"case {t}: row {row}: {worst:.3g}"
        empty = np.diff(rp) == 0
        assert Cg[empty].tobytes() == C0[empty].tobytes(), t


@pytest.mark.parametrize("config", [1, 2, 3, 4, 5])
def test_workloads_row_sample(orc, config):
    """The five workloads at their full benchmark sizes, checked on a seeded sample of 3000 rows
    against the oracle."""
    import torch
    size = 0
    w = vm.WORKLOADS[config]
    fp32 = w["precision"] == "fp32"
    A = vm.generate(config, size)
    O = w["O"]
    B = vm.dense(A.N, O, seed=vm.SEED_BASE + 100 + config, fp16_exact=not fp32)
    say("workload", config, size, A.M, A.nnz, O)
    with vm.DeviceFormat.from_device_csr(dev(A.row_ptr), dev(A.col), dev(A.val), A.M, A.N,
                                         fp32, 32) as f:
        dB = dev(B).half() if not fp32 else dev(B)
        C = torch.zeros((A.M, O), dtype=torch.float32, device="cuda")
        f.spmm(dB, C, tileK=128)
        Cn = C.cpu().numpy()
        scale = f.info()["scale"]
    rng = np.random.default_rng(config)
    rows = np.sort(rng.choice(A.M, size=min(A.M, 3000), replace=False))
    srp, sc, sv = sub_csr(A.row_ptr, A.col, A.val, rows)
    R, L1 = orc.spmm_csr(srp, sc, sv, len(rows), B, mode=0 if fp32 else 1, scale=scale)
    ok, worst, row = row_l1_parity(Cn[rows], R, L1, TAU[fp32])
    assert ok, f"row {rows[row]}: {worst:.3g}"


@pytest.mark.parametrize("config", [2, 3, 4])
def test_workload_upload_path(config):
    """The reference's upload_vcsr_mc_device path at full size: the format arrays a build returns
    (csr_to_vcsr_mc's output), uploaded back (vcsrmc_upload validates them on the device and
    derives the execution layout from them), give the same layout and, with no split panels
    (no atomics), the same C bit for bit as the format built from the CSR, in both launch modes
    -- so the row-sample parity of the build path holds for the upload path too."""
    import torch
    w = vm.WORKLOADS[config]
    fp32 = w["precision"] == "fp32"
    A = vm.generate(config, 0)
    O = w["O"]
    B = vm.dense(A.N, O, seed=vm.SEED_BASE + 300 + config, fp16_exact=not fp32)
    dB = dev(B) if fp32 else dev(B).half()
    say("workload upload path", config, A.M, A.nnz, O)
    with vm.DeviceFormat.from_device_csr(dev(A.row_ptr), dev(A.col), dev(A.val), A.M, A.N,
                                         fp32, 32) as f:
        V = f.download()
        built = f.info()
        assert built["num_split_panels"] == 0, built
        want = []
        for overwrite in (False, True):
            C = torch.zeros((A.M, O), dtype=torch.float32, device="cuda") + 0.5
            f.spmm(dB, C, tileK=128, overwrite=overwrite)
            want.append(C)
    with vm.DeviceFormat.from_host_format(V) as g:
        assert g.info() == built
        for overwrite, Cw in zip((False, True), want):
            C = torch.zeros((A.M, O), dtype=torch.float32, device="cuda") + 0.5
            g.spmm(dB, C, tileK=128, overwrite=overwrite)
            torch.cuda.synchronize()
            assert torch.equal(C, Cw), overwrite


@pytest.mark.parametrize("config", [1, 2, 3, 4, 5])
def test_workloads_second_precision_row_sample(orc, config):
    """The reference's driver runs both kernels on every matrix (src/main.cpp:345): each
    workload at full size in the precision it is not configured for -- vcsr_mc_fp32 for the
    FP16 workloads, vcsr_mc for the FP32 ones, fed FP32 B as the reference's
    run_vcsr_mc_spmm_gpu is -- on a seeded sample of 2000 rows against the oracle."""
    import torch
    w = vm.WORKLOADS[config]
    fp32 = w["precision"] != "fp32"
    A = vm.generate(config, 0)
    O = w["O"]
    B = vm.dense(A.N, O, seed=vm.SEED_BASE + 200 + config)
    say("workload second precision", config, A.M, A.nnz, O, "fp32" if fp32 else "fp16")
    with vm.DeviceFormat.from_device_csr(dev(A.row_ptr), dev(A.col), dev(A.val), A.M, A.N,
                                         fp32, 32) as f:
        C = torch.zeros((A.M, O), dtype=torch.float32, device="cuda")
        f.spmm(dev(B), C, tileK=128)
        rows = np.sort(np.random.default_rng(100 + config).choice(A.M, size=min(A.M, 2000),
                                                                  replace=False))
        Cs = C[torch.from_numpy(rows).cuda()].cpu().numpy()
        scale = f.info()["scale"]
    srp, sc, sv = sub_csr(A.row_ptr, A.col, A.val, rows)
    R, L1 = orc.spmm_csr(srp, sc, sv, len(rows), B, mode=0 if fp32 else 1, scale=scale)
    ok, worst, row = row_l1_parity(Cs, R, L1, TAU[fp32])
    assert ok, f"row {rows[row]}: {worst:.3g}"


@pytest.mark.parametrize("config,tileK", [(1, 128), (2, 128), (3, 128), (4, 128), (4, 64),
                                           (2, 32)])
def test_workloads_full_size_accumulate_twice(config, tileK):
    """At the full benchmark sizes, a property exact at any size: with no split panel (no
    atomics) every output is one rounding of the same deterministic sum into C, so from
    C = -0.0 one call leaves s and a second exactly 2 s; rows without nonzeros are never
    written, so they keep the sign of -0.0."""
    import torch
    w = vm.WORKLOADS[config]
    fp32 = w["precision"] == "fp32"
    A = vm.generate(config, 0)
    O = w["O"]
    say("full-size accumulate twice", config, tileK, A.M, A.nnz, O)
    g = torch.Generator(device="cuda")
    g.manual_seed(config)
    B = torch.rand((A.N, O), generator=g, device="cuda") * 2 - 1
    dB = B if fp32 else B.half()
    with vm.DeviceFormat.from_device_csr(dev(A.row_ptr), dev(A.col), dev(A.val), A.M, A.N,
                                         fp32, 32) as f:
        info = f.info()
        assert info["num_units"] == info["num_panels"]  # no split panel
        C1 = torch.full((A.M, O), -0.0, dtype=torch.float32, device="cuda")
        f.spmm(dB, C1, tileK=tileK)
        C2 = C1.clone()
        f.spmm(dB, C2, tileK=tileK)
        torch.cuda.synchronize()
    assert torch.equal(C2, 2 * C1)
    empty = torch.from_numpy(np.diff(A.row_ptr) == 0).cuda()
    assert bool(torch.all(torch.signbit(C2[empty])) and torch.all(C2[empty] == 0))
    assert bool(torch.isfinite(C1).all())
    assert int((C1[~empty] != 0).any(dim=1).sum()) == int((~empty).sum())


@pytest.mark.parametrize("fp32,b32", [(False, False), (True, True), (False, True)])
def test_graph_replay(fp32, b32):
    """The multiply launch captured in a HIP graph (no allocation or memset inside it) replays
    to the eager result, several times, with eager work and synchronisation between replays.
    An FP16 format given FP32 B allocates its conversion buffer on first use, so that case is
    called once before capture."""
    import torch
    rng = np.random.default_rng(21)
    rp, c, v = random_csr(rng, 700, 500, nnz_per_row=9, heavy_rows=3, heavy_nnz=450)
    B = rng.uniform(-1, 1, (500, 96)).astype(np.float32)
    say("graph replay", fp32, b32)
    with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), 700, 500, fp32, 32) as f:
        dB = dev(B) if (fp32 or b32) else dev(B).half()
        ref = torch.zeros((700, 96), dtype=torch.float32, device="cuda")
        f.spmm(dB, ref, tileK=64)
        torch.cuda.synchronize()
        C = torch.zeros_like(ref)
        stream = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            f.spmm(dB, C, tileK=64, stream=stream)
        for it in range(4):
            C.zero_()
            junk = torch.randn(1000, device="cuda").sum()  # eager work between replays
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert float(junk) == float(junk)
            got, want = C.cpu().numpy(), ref.cpu().numpy()
            # split panels merge with atomics: only their order may differ
            assert np.allclose(got, want, rtol=1e-6, atol=1e-6), it


def _split_rows(rp, c, M, N, light_max=1, heavy_tiles=64):
    """Rows of the 16-row panels that the format cuts into several heavy units (a panel of
    more than heavy_tiles 32-column tiles, for formats of fewer than 2048 panels)."""
    rows = np.repeat(np.arange(M), np.diff(rp))
    panel = rows // 16
    keys = np.unique(panel.astype(np.int64) * (N + 1) + c)
    tiles = (np.bincount(keys // (N + 1), minlength=(M + 15) // 16) + 31) // 32
    split = np.nonzero((tiles > light_max) & (tiles > heavy_tiles))[0]
    out = np.zeros(M, bool)
    for p in split:
        out[16 * p:16 * p + 16] = True
    return out


@pytest.mark.parametrize("fp32", [False, True])
@pytest.mark.parametrize("tileK", [32, 128])
@pytest.mark.parametrize("O", [7, 128])
def test_overwrite_equals_zero_then_accumulate(orc, fp32, tileK, O):
    """C = A.B (the overwrite flag, C never read) against C zeroed and C += A.B: bit for bit on
    every row outside split panels; split panels (several units adding through atomics into
    rows the launcher clears first) within the parity norm of the oracle.  Rows without
    nonzeros keep what C held, bit for bit.  The layout is kept in natural row order, where
    _split_rows knows which panels are split (row maps: tests/test_gpu_row_groups.py)."""
    import torch
    rng = np.random.default_rng(31 + tileK + O + fp32)
    M, N = 900, 5000
    rp, c, v = random_csr(rng, M, N, density=0.001, heavy_rows=5, heavy_nnz=4000,
                          empty_frac=0.3)
    B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
    split = _split_rows(rp, c, M, N)
    assert split.any()
    say("overwrite vs accumulate", fp32, tileK, O)
    vm.set_row_grouping(vm.ROW_GROUPING_OFF)
    try:
        f = vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, N, fp32, 32)
    finally:
        vm.set_row_grouping(vm.ROW_GROUPING_AUTO)
    assert f.info()["row_grouped"] == 0
    assert f.info()["num_split_panels"] == np.unique(np.nonzero(split)[0] // 16).size
    with f:
        dB = dev(B) if fp32 else dev(B).half()
        Ca = torch.zeros((M, O), dtype=torch.float32, device="cuda")
        f.spmm(dB, Ca, tileK=tileK)
        C0 = rng.uniform(5, 6, (M, O)).astype(np.float32)
        Co = dev(C0)
        f.spmm(dB, Co, tileK=tileK, overwrite=True)
        Co2 = Co.clone()
        f.spmm(dB, Co2, tileK=tileK, overwrite=True)  # idempotent
        torch.cuda.synchronize()
        scale = f.info()["scale"]
        Ca, Co, Co2 = Ca.cpu().numpy(), Co.cpu().numpy(), Co2.cpu().numpy()
    empty = np.diff(rp) == 0
    keep = ~split & ~empty
    assert Co[keep].tobytes() == Ca[keep].tobytes()
    assert Co2[keep].tobytes() == Ca[keep].tobytes()
    assert Co[empty].tobytes() == C0[empty].tobytes()
    R, L1 = orc.spmm_csr(rp, c, v, M, B, mode=0 if fp32 else 1, scale=scale)
    for C in (Co, Co2):
        ok, worst, row = row_l1_parity(C[~empty], R[~empty], L1[~empty], TAU[fp32])
        assert ok, f"row {row}: {worst:.3g}"


def test_overwrite_unaligned_c(orc):
    """Overwrite with C not 16-byte aligned (scalar epilogue) and O not a multiple of 4."""
    import torch
    rng = np.random.default_rng(33)
    M, N, O = 400, 300, 13
    rp, c, v = random_csr(rng, M, N, density=0.02, empty_frac=0.2)
    B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
    say("overwrite unaligned")
    with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, N, True, 32) as f:
        buf = torch.full((M * O + 1,), 3.0, dtype=torch.float32, device="cuda")
        Cv = buf[1:]
        f.spmm(dev(B), Cv, tileK=16, O=O, overwrite=True)
        torch.cuda.synchronize()
        got = Cv.cpu().numpy().reshape(M, O)
    R, L1 = orc.spmm_csr(rp, c, v, M, B, mode=0)
    empty = np.diff(rp) == 0
    assert np.all(got[empty] == 3.0)
    ok, worst, row = row_l1_parity(got[~empty], R[~empty], L1[~empty], TAU[True])
    assert ok, f"row {row}: {worst:.3g}"


@pytest.mark.parametrize("config", [1, 2, 4, 5])
def test_workloads_full_size_overwrite(orc, config):
    """Full benchmark sizes: the overwrite launch equals zero-then-accumulate bit for bit outside
    split panels (R-MAT has a few), and a seeded sample of 2000 rows meets the parity norm."""
    import torch
    w = vm.WORKLOADS[config]
    fp32 = w["precision"] == "fp32"
    A = vm.generate(config, 0)
    O = w["O"]
    B = vm.dense(A.N, O, seed=vm.SEED_BASE + 100 + config, fp16_exact=not fp32)
    say("full-size overwrite", config, A.M, A.nnz, O)
    with vm.DeviceFormat.from_device_csr(dev(A.row_ptr), dev(A.col), dev(A.val), A.M, A.N,
                                         fp32, 32) as f:
        info = f.info()
        dB = dev(B) if fp32 else dev(B).half()
        Ca = torch.zeros((A.M, O), dtype=torch.float32, device="cuda")
        f.spmm(dB, Ca, tileK=128)
        Co = torch.full((A.M, O), 9.0, dtype=torch.float32, device="cuda")
        f.spmm(dB, Co, tileK=128, overwrite=True)
        torch.cuda.synchronize()
        empty = torch.from_numpy(np.diff(A.row_ptr) == 0).cuda()
        assert bool(torch.all(Co[empty] == 9.0))
        if info["num_units"] == info["num_panels"]:  # no split panel
            assert torch.equal(Co[~empty], Ca[~empty])
        else:
            assert bool(torch.allclose(Co[~empty], Ca[~empty], rtol=1e-5, atol=1e-5))
        rows = np.sort(np.random.default_rng(config).choice(A.M, size=min(A.M, 2000),
                                                            replace=False))
        Cs = Co[torch.from_numpy(rows).cuda()].cpu().numpy()
        scale = info["scale"]
    srp, sc, sv = sub_csr(A.row_ptr, A.col, A.val, rows)
    R, L1 = orc.spmm_csr(srp, sc, sv, len(rows), B, mode=0 if fp32 else 1, scale=scale)
    ne = np.diff(srp) > 0
    ok, worst, row = row_l1_parity(Cs[ne], R[ne], L1[ne], TAU[fp32])
    assert ok, f"row {row}: {worst:.3g}"


def test_failed_conversion_allocation_leaves_handle_usable(orc):
    """An FP16 format given FP32 B converts B into a buffer its handle allocates on first use.
    When that allocation fails (N x O binary16 values far beyond the GPU's memory; nothing is
    launched, since the conversion follows the allocation) the call returns the HIP error and
    the handle stays usable: the next call allocates again and meets the parity norm."""
    import torch
    rng = np.random.default_rng(51)
    M = N = 2000
    rp, c, v = random_csr(rng, M, N, nnz_per_row=16)
    assert len(c) >= 12 * N  # with B above 256 MB the launcher converts
    O_huge = 2**31 - 1
    total = torch.cuda.get_device_properties(0).total_memory
    assert N * O_huge * 2 > 10 * total
    O = 128
    B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
    say("failed conversion allocation")
    with vm.DeviceFormat.from_device_csr(dev(rp), dev(c), dev(v), M, N, False, 32) as f:
        dB = dev(B)
        C = torch.zeros((M, O), dtype=torch.float32, device="cuda")
        stream = int(torch.cuda.current_stream().cuda_stream)
        rc = vm.lib().vcsrmc_spmm(f.handle, dB.data_ptr(), vm.B_F32, O_huge, 128, C.data_ptr(),
                                  stream, None)
        assert rc == vm.ERR_HIP and b"hipMalloc" in vm.lib().vcsrmc_last_error()
        torch.cuda.synchronize()
        assert bool(torch.all(C == 0))
        f.spmm(dB, C, tileK=128)
        torch.cuda.synchronize()
        Cn = C.cpu().numpy()
        scale = f.info()["scale"]
    R, L1 = orc.spmm_csr(rp, c, v, M, B, mode=1, scale=scale)
    ok, worst, row = row_l1_parity(Cn, R, L1, TAU[False])
    assert ok, f"row {row}: {worst:.3g}"


@pytest.mark.parametrize("fp32", [False, True])
@pytest.mark.parametrize("O", [1024, 1500, 2048])
def test_wide_o(orc, fp32, O):
    """Wide B and C: 8 or more O tiles, so every XCD group takes its own O tile and the rest
    become launch rows (O = 2048: 16 tiles of 128), with O not a multiple of the tile width
    (1500), C starting non-zero."""
    rng = np.random.default_rng(O + fp32)
    M, N = 700, 900
    rp, c, v = random_csr(rng, M, N, density=0.01, heavy_rows=2, heavy_nnz=600,
                          empty_frac=0.1)
    B = rng.uniform(-1, 1, (N, O)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, O)).astype(np.float32)
    say("wide O", fp32, O)
    check(orc, rp, c, v, M, N, B, fp32, tileK=128, C0=C0)
