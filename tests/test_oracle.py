"""Pins the CPU oracle (oracle/) before anything is compared with it.

Each check is chosen so that a plausible slip in the restatement (a dropped term, a wrong
index, a transposed operand, a wrong tie or rounding rule) fails at least one of them:
  * float16 conversion: against numpy's independent IEEE conversion, exhaustively;
  * half_scale: closed forms, and against the reference's own compiled function;
  * builder: against the reference's own csr_to_vcsr_mc (oracle/_ref, here) and the committed
    fixtures it wrote (everywhere), plus closed forms and invariants;
  * SpMM: against a dense float64 numpy product of the same quantised operands.
"""
import numpy as np
import pytest

from conftest import random_csr
from golden_io import load_cases

pytestmark = []


# ---- float16 -------------------------------------------------------------------------------
def test_f16_all_halves_roundtrip(orc):
    h = np.arange(65536, dtype=np.uint16)
    f = h.view(np.float16).astype(np.float32)
    bits = orc.f32_to_f16_bits(f)
    nan = np.isnan(f)
    assert np.array_equal(bits[~nan], h[~nan])
    assert np.all((bits[nan] & 0x7c00) == 0x7c00) and np.all(bits[nan] & 0x3ff)


def test_f16_rounding_matches_numpy(orc):
    rng = np.random.default_rng(1)
    # random bit patterns over the whole float range, plus every midpoint between adjacent halves
    x = rng.integers(0, 2**32, size=400000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    h = np.arange(0, 0x7bff, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mids = ((lo + hi) / 2).astype(np.float32)
    edges = np.array([65504, 65519.99, 65520, 65536, 6.1035156e-05, 5.96e-08, 2.98e-08,
                      2.9802322e-08, 1e-10, -0.0, 0.0], np.float32)
    for arr in (x, mids, -mids, edges):
        ok = ~np.isnan(arr)
        got = orc.f32_to_f16_bits(arr[ok])
        with np.errstate(over="ignore"):
            want = arr[ok].astype(np.float16).view(np.uint16)
        assert np.array_equal(got, want)


# ---- half_scale ----------------------------------------------------------------------------
@pytest.mark.parametrize("amax,expect", [
    (0.0, 1.0), (1.0, 1.0), (60000.0, 1.0), (6.103515625e-05, 1.0),
    (1e5, np.float32(1e5) * (np.float32(1) / np.float32(60000))),
    (6e-5, np.float32(6e-5) * (np.float32(1) / np.float32(60000))),
    (np.inf, np.inf),
])
def test_half_scale_closed_form(orc, amax, expect):
    v = np.array([0.5 * amax, -amax, 0.25], np.float32) if amax > 0.25 else \
        np.array([-amax, 0.5 * amax], np.float32)
    assert np.float32(orc.half_scale(v)).tobytes() == np.float32(expect).tobytes()


def test_half_scale_matches_reference_binary(orc):
    if not orc.ref_available():
        pytest.skip("oracle/_ref is built only where the reference sources are")
    rng = np.random.default_rng(2)
    xs = np.concatenate([rng.uniform(6e4, 1e9, 3000), rng.uniform(1e-12, 6.1e-5, 3000),
                         rng.uniform(-2, 2, 100)]).astype(np.float32)
    for x in xs:
        v = np.array([x, -0.5 * x], np.float32)
        assert orc.half_scale(v).tobytes() == orc.ref_half_scale(v).tobytes()


# ---- builder -------------------------------------------------------------------------------
def _build(orc, rp, c, v, M, N, segw, fp32):
    return orc.build_format(rp, c, v, M, N, segw, fp32)


def test_builder_matches_golden_fixtures(orc):
    for case in load_cases():
        f = _build(orc, case["row_ptr"], case["col"], case["val"], case["M"], case["N"],
                   case["segw"], case["fp32"])
        ref = orc.canonicalize(orc.Format(case["ref"]))
        assert orc.formats_equal(f, ref) == [], case["name"]


def test_builder_matches_reference_random(orc):
    if not orc.ref_available():
        pytest.skip("oracle/_ref is built only where the reference sources are")
    rng = np.random.default_rng(3)
    for t in range(40):
        M, N = int(rng.integers(1, 400)), int(rng.integers(1, 400))
        rp, c, v = random_csr(rng, M, N, density=float(rng.choice([0.005, 0.03, 0.2, 0.7])),
                              mag=float(rng.choice([1.0, 1e5, 1e-5])), empty_frac=0.2)
        for segw in (16, 32, 48, 64):
            fp32 = bool(rng.integers(0, 2))
            a = _build(orc, rp, c, v, M, N, segw, fp32)
            b = orc.canonicalize(orc.ref_build_format(rp, c, v, M, N, segw, fp32))
            assert orc.formats_equal(a, b) == [], (t, M, N, segw, fp32)


@pytest.mark.parametrize("M,per_row,segw", [(16384, 8, 16), (70000, 30, 16)])
def test_builder_matches_reference_multi_group_items(orc, M, per_row, segw):
    """G >= 8192 (chunk = 2) and G >= 131072 (chunk = 32) work items."""
    if not orc.ref_available():
        pytest.skip("oracle/_ref is built only where the reference sources are")
    rng = np.random.default_rng(M)
    rp = np.zeros(M + 1, np.int32)
    k = rng.poisson(per_row, M).clip(0, M)
    rp[1:] = np.cumsum(k)
    col = np.concatenate([np.sort(rng.choice(M, size=int(x), replace=False)) for x in k])
    col = col.astype(np.int32)
    val = rng.uniform(-1, 1, col.size).astype(np.float32)
    a = _build(orc, rp, col, val, M, M, segw, False)
    G = len(a["group_depth"])
    chunk = max(1, min(32, G // 4096))
    assert chunk >= 2
    b = orc.canonicalize(orc.ref_build_format(rp, col, val, M, M, segw, False))
    assert orc.formats_equal(a, b) == []


def test_builder_closed_forms(orc):
    # diagonal n x n, segw 16: segment s holds rows 16s..16s+15, one group of depth 1 each
    n = 37
    rp, c = np.arange(n + 1, dtype=np.int32), np.arange(n, dtype=np.int32)
    v = np.linspace(-1, 1, n).astype(np.float32)
    f = _build(orc, rp, c, v, n, n, 16, True)
    S = (n + 15) // 16
    assert f["num_segments"] == S and len(f["group_depth"]) == S
    assert np.all(f["group_depth"] == 1)
    assert np.array_equal(f["group_seg_base"], 16 * np.arange(S))
    assert np.array_equal(f["group_ptr"], 16 * np.arange(S + 1))
    rows = f["group_rows"].reshape(S, 16)
    for s in range(S):
        want = [r for r in range(16 * s, min(16 * s + 16, n))]
        assert list(rows[s][: len(want)]) == want and np.all(rows[s][len(want):] == -1)
    # one dense 32 x 32 block at block column 1 of a 32 x 64 matrix, segw 32: depth 32
    rp = (32 * np.arange(33)).astype(np.int32)
    c = np.tile(np.arange(32, 64), 32).astype(np.int32)
    v = np.arange(1024, dtype=np.float32)
    f = _build(orc, rp, c, v, 32, 64, 32, False)
    assert list(f["group_depth"]) == [32, 32] and list(f["group_seg_base"]) == [32, 32]
    lc = f["lcol"].reshape(2, 32, 16)  # group, depth, lane
    assert np.array_equal(lc[0], np.tile(np.arange(32)[:, None], (1, 16)))
    # nnz = 0
    f = _build(orc, np.zeros(4, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32), 3, 5,
               16, False)
    assert len(f["group_depth"]) == 0 and list(f["group_ptr"]) == [0] and len(f["item_gbeg"]) == 0


def test_builder_invariants(orc, rng):
    for t in range(10):
        M, N = int(rng.integers(1, 300)), int(rng.integers(1, 300))
        rp, c, v = random_csr(rng, M, N, density=0.05, empty_frac=0.1)
        segw = int(rng.choice([16, 32, 48, 64]))
        f = _build(orc, rp, c, v, M, N, segw, False)
        G = len(f["group_depth"])
        assert np.array_equal(np.diff(f["group_ptr"]), 16 * f["group_depth"])
        seen = set()
        for g in range(G):
            base, d = f["group_ptr"][g], f["group_depth"][g]
            rows = f["group_rows"][16 * g: 16 * g + 16]
            counts = []
            for lane in range(16):
                lc = f["lcol"][base + 16 * np.arange(d) + lane]
                vv = f["val"][base + 16 * np.arange(d) + lane]
                k = int(np.sum(lc >= 0))
                assert np.all(lc[:k] >= 0) and np.all(lc[k:] == -1) and np.all(vv[k:] == 0)
                if rows[lane] < 0:
                    assert k == 0
                    continue
                counts.append(k)
                for dd in range(k):
                    cc = f["group_seg_base"][g] + lc[dd]
                    seen.add((int(rows[lane]), int(cc)))
            assert max(counts) == d                       # depth = max count in the bundle
            assert counts == sorted(counts, reverse=True)  # non-increasing inside a bundle
        want = {(r, int(c[p])) for r in range(M) for p in range(rp[r], rp[r + 1])}
        assert seen == want                                # every nonzero exactly once
        # items partition [0, G) in runs of one segment, sorted by work, descending
        ib, ie = f["item_gbeg"], f["item_gend"]
        assert sorted(zip(ib, ie)) == sorted(zip(ib, ie)) and sum(ie - ib) == G
        work = f["group_ptr"][ie] - f["group_ptr"][ib]
        assert np.all(np.diff(work) <= 0)


def test_canonicalize_detects_planted_swap(orc):
    """A format with two rows swapped across a count boundary is not canonical-equal."""
    rng = np.random.default_rng(5)
    rp, c, v = random_csr(rng, 64, 64, density=0.2)
    f = _build(orc, rp, c, v, 64, 64, 16, False)
    bad = orc.Format({k: (np.array(x, copy=True) if isinstance(x, np.ndarray) else x)
                      for k, x in f.items()})
    lc = bad["lcol"]
    j = next(j for j in range(1, 16) if lc[j] >= 0 and lc[j] != lc[0])
    lc[0], lc[j] = lc[j], lc[0]
    assert "lcol" in orc.formats_equal(orc.canonicalize(bad), f)
    B = rng.uniform(-1, 1, (64, 8)).astype(np.float32)
    assert not np.allclose(orc.spmm_format(bad, B), orc.spmm_format(f, B))


def test_canonicalize_idempotent_and_keeps_invariants(orc, rng):
    if not orc.ref_available():
        pytest.skip("oracle/_ref is built only where the reference sources are")
    rp, c, v = random_csr(rng, 500, 500, density=0.03)
    r = orc.ref_build_format(rp, c, v, 500, 500, 32, False)
    a = orc.canonicalize(r)
    for k in ("group_ptr", "group_depth", "group_seg_base", "item_gbeg", "item_gend"):
        assert np.array_equal(a[k], r[k])
    assert orc.formats_equal(orc.canonicalize(a), a) == []


# ---- SpMM ----------------------------------------------------------------------------------
def _dense(rp, c, v, M, N):
    A = np.zeros((M, N), np.float64)
    for r in range(M):
        A[r, c[rp[r]:rp[r + 1]]] = v[rp[r]:rp[r + 1]]
    return A


def test_spmm_fp32_matches_dense(orc, rng):
    rp, c, v = random_csr(rng, 60, 70, density=0.1)
    B = rng.uniform(-1, 1, (70, 13)).astype(np.float32)
    R, L1 = orc.spmm_csr(rp, c, v, 60, B, mode=0)
    A = _dense(rp, c, v, 60, 70)
    np.testing.assert_allclose(R, A @ B.astype(np.float64), rtol=0, atol=1e-12)
    np.testing.assert_allclose(L1, (np.abs(A) @ np.abs(B.astype(np.float64))).sum(1), rtol=1e-12)


def test_spmm_fp16_model_matches_dense(orc, rng):
    rp, c, v = random_csr(rng, 50, 40, density=0.2, mag=1e5)
    B = rng.uniform(-3, 3, (40, 9)).astype(np.float32)
    s = orc.half_scale(v)
    assert s != 1.0
    R, _ = orc.spmm_csr(rp, c, v, 50, B, mode=1, scale=s)
    inv = np.float32(1) / np.float32(s)
    a16 = (v * inv).astype(np.float32).astype(np.float16).astype(np.float64)
    b16 = B.astype(np.float16).astype(np.float64)
    want = _dense(rp, c, a16, 50, 40) @ b16 * np.float64(s)
    np.testing.assert_allclose(R, want, rtol=1e-12, atol=1e-9)


def test_spmm_format_equals_csr(orc, rng):
    for fp32 in (False, True):
        rp, c, v = random_csr(rng, 90, 110, density=0.07)
        B = rng.uniform(-1, 1, (110, 17)).astype(np.float32)
        f = _build(orc, rp, c, v, 90, 110, 32, fp32)
        R1 = orc.spmm_format(f, B)
        R2, L1 = orc.spmm_csr(rp, c, v, 90, B, mode=0 if fp32 else 1, scale=float(f["scale"]))
        assert np.all(np.abs(R1 - R2).sum(1) <= 1e-12 * (L1 + 1e-300))


def test_cpu_baseline_loop_matches_dense(orc, rng):
    rp, c, v = random_csr(rng, 40, 30, density=0.2)
    B = rng.uniform(-1, 1, (30, 6)).astype(np.float32)
    R = orc.cpu_spmm_f64(rp, c, v, B)
    np.testing.assert_allclose(R, _dense(rp, c, v, 40, 30) @ B.astype(np.float64), atol=1e-12)
    R2 = orc.cpu_spmm_f64(rp, c, v, B, threads=4)
    assert R2.tobytes() == R.tobytes()


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("with_c0", [False, True])
def test_spmm_check_equals_spmm_csr(orc, rng, mode, with_c0):
    """The whole-matrix check gives, per row, exactly |C - (R + C0)|_1 and rowL1 + |C0|_1 of
    spmm_csr (the same arithmetic, row by row), and with norms=True |R + C0|_1, |C - (R + C0)|_2^2
    and |R + C0|_2^2, at one and at several threads; a planted error in one element of C moves
    that row's error and no other."""
    rp, c, v = random_csr(rng, 300, 200, density=0.05, empty_frac=0.2, mag=1e5 if mode else 1)
    B = rng.uniform(-2, 2, (200, 19)).astype(np.float32)  # not binary16-exact: mode 1 rounds it
    s = float(orc.half_scale(v)) if mode else 1.0
    R, L1 = orc.spmm_csr(rp, c, v, 300, B, mode=mode, scale=s)
    C0 = rng.uniform(-1, 1, R.shape).astype(np.float32) if with_c0 else None
    want = R + (C0.astype(np.float64) if with_c0 else 0.0)
    C = (want + rng.normal(0, 1e-3, R.shape)).astype(np.float32)
    # sums in index order, as the check forms them (numpy's sum is pairwise)
    err_want = np.cumsum(np.abs(C.astype(np.float64) - want), axis=1)[:, -1]
    bound_want = L1 + (np.cumsum(np.abs(C0.astype(np.float64)), axis=1)[:, -1] if with_c0
                       else 0.0)
    d = C.astype(np.float64) - want
    norms_want = [np.cumsum(x, axis=1)[:, -1] for x in (np.abs(want), d * d, want * want)]
    for threads in (1, 5):
        err, bound = orc.spmm_check(rp, c, v, 300, B, C, mode=mode, scale=s, C0=C0,
                                    threads=threads)
        assert err.tobytes() == err_want.tobytes()
        assert bound.tobytes() == bound_want.tobytes()
        out = orc.spmm_check(rp, c, v, 300, B, C, mode=mode, scale=s, C0=C0, threads=threads,
                             norms=True)
        assert len(out) == 5
        for got, ref in zip(out, [err_want, bound_want] + norms_want):
            assert got.tobytes() == ref.tobytes()
    C2 = C.copy()
    C2[17, 3] += 0.5
    err2, _ = orc.spmm_check(rp, c, v, 300, B, C2, mode=mode, scale=s, C0=C0, threads=3)
    moved = np.nonzero(err2 != err)[0]
    assert moved.tolist() == [17] and err2[17] > err[17] + 0.49
