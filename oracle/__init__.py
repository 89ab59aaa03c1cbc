"""ctypes binding of the CPU oracle (test infrastructure only).

Only the test suite, ``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py``
import this package.  The product library never loads it.  What each function restates
(file:line of MuuSeoTia/VCSR_MC) and how it is pinned is written in ``vcsrmc_oracle.h``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libvcsrmc_oracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libvcsrmc_ref.so")
REFERENCE_ROOT = "/root/reference"


class OrcFormat(C.Structure):
    _fields_ = [
        ("M", C.c_int), ("N", C.c_int), ("segw", C.c_int), ("bundle", C.c_int),
        ("num_segments", C.c_int), ("G", C.c_int), ("nval", C.c_longlong), ("nitems", C.c_int),
        ("group_ptr", C.POINTER(C.c_int)), ("group_depth", C.POINTER(C.c_int)),
        ("group_seg_base", C.POINTER(C.c_int)), ("group_rows", C.POINTER(C.c_int)),
        ("lcol", C.POINTER(C.c_int)), ("val", C.POINTER(C.c_float)),
        ("item_gbeg", C.POINTER(C.c_int)), ("item_gend", C.POINTER(C.c_int)),
        ("scale", C.c_float), ("fp32", C.c_int),
    ]


ARRAYS = ("group_ptr", "group_depth", "group_seg_base", "group_rows", "lcol", "val",
          "item_gbeg", "item_gend")


def build(force: bool = False, ref: bool | None = None) -> None:
    """Compile the oracle (and, where the reference sources exist, oracle/_ref)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)
    if ref is None:
        ref = os.path.isdir(os.path.join(REFERENCE_ROOT, "src"))
    if ref and (force or not os.path.exists(REF_PATH)):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        i32p, f32p, f64p = C.POINTER(C.c_int), C.POINTER(C.c_float), C.POINTER(C.c_double)
        L.orc_half_scale.restype = C.c_float
        L.orc_half_scale.argtypes = [f32p, C.c_longlong]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_f16_array.argtypes = [f32p, C.POINTER(C.c_uint16), C.c_longlong]
        L.orc_round_f16_array.argtypes = [f32p, f32p, C.c_longlong]
        L.orc_build.restype = C.c_int
        L.orc_build.argtypes = [i32p, i32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                                C.POINTER(OrcFormat)]
        L.orc_free.argtypes = [C.POINTER(OrcFormat)]
        L.orc_canonicalize.restype = C.c_int
        L.orc_canonicalize.argtypes = [C.POINTER(OrcFormat)]
        L.orc_spmm_csr.argtypes = [i32p, i32p, f32p, C.c_int, f32p, C.c_int, C.c_int, C.c_float,
                                   f64p, f64p]
        L.orc_spmm_format.argtypes = [C.POINTER(OrcFormat), f32p, C.c_int, f64p]
        L.orc_spmm_check.restype = C.c_int
        L.orc_spmm_check.argtypes = [i32p, i32p, f32p, C.c_int, f32p, C.c_longlong, C.c_int,
                                     C.c_int, C.c_float, f32p, f32p, C.c_int, f64p, f64p, f64p, f64p,
                                     f64p]
        L.orc_cpu_spmm_f64.argtypes = [i32p, i32p, f32p, C.c_int, f32p, C.c_int, f64p]
        L.orc_cpu_spmm_f64_rows.argtypes = [i32p, i32p, f32p, C.c_int, C.c_int, f32p, C.c_int, f64p]
        L.orc_cpu_spmm_f64_omp.argtypes = [i32p, i32p, f32p, C.c_int, C.c_int, f32p, C.c_int, f64p,
                                           C.c_int]
        L.orc_std_sort_by_key.argtypes = [i32p, C.c_longlong, i32p]
        L.orc_heap_sort_by_key.argtypes = [i32p, C.c_longlong, i32p]
        L.orc_rcm_order.restype = C.c_int
        L.orc_rcm_order.argtypes = [i32p, i32p, C.c_int, C.c_int, i32p]
        L.orc_apply_column_permutation.restype = C.c_int
        L.orc_apply_column_permutation.argtypes = [i32p, i32p, f32p, C.c_int, C.c_int, i32p, f32p,
                                                   C.c_int, f32p]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref_lib():
    global _ref
    if _ref is None:
        R = C.CDLL(REF_PATH)
        R.ref_build.restype = C.c_int
        R.ref_build.argtypes = [C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_float),
                                C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(OrcFormat),
                                C.c_char_p, C.c_int]
        R.ref_half_scale.restype = C.c_float
        R.ref_half_scale.argtypes = [C.POINTER(C.c_float), C.c_int]
        i32p, f32p = C.POINTER(C.c_int), C.POINTER(C.c_float)
        R.ref_std_sort_by_key.argtypes = [i32p, C.c_longlong, i32p]
        R.ref_partial_sort_by_key.argtypes = [i32p, C.c_longlong, i32p]
        R.ref_sort_adversary.argtypes = [C.c_int, i32p]
        R.ref_rcm_order.argtypes = [i32p, i32p, C.c_int, C.c_int, i32p]
        R.ref_apply_column_permutation.argtypes = [i32p, i32p, f32p, C.c_int, C.c_int, i32p, f32p,
                                                   C.c_int]
        R.ref_spmm_gpu.restype = C.c_int
        R.ref_spmm_gpu.argtypes = [i32p, i32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                                   C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_char_p, C.c_int]
        _ref = R
    return _ref


def _p(a, ct):
    return a.ctypes.data_as(C.POINTER(ct))


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class Format(dict):
    """A VCSRMC format as a dict of numpy arrays plus scalar fields."""


def _take(f: OrcFormat) -> Format:
    out = Format(M=f.M, N=f.N, segw=f.segw, bundle=f.bundle, num_segments=f.num_segments,
                 scale=np.float32(f.scale), fp32=bool(f.fp32))
    sizes = dict(group_ptr=f.G + 1, group_depth=f.G, group_seg_base=f.G, group_rows=16 * f.G,
                 lcol=f.nval, val=f.nval, item_gbeg=f.nitems, item_gend=f.nitems)
    for name in ARRAYS:
        n = sizes[name]
        ptr = getattr(f, name)
        dt = np.float32 if name == "val" else np.int32
        out[name] = np.ctypeslib.as_array(ptr, shape=(n,)).astype(dt, copy=True) if n else \
            np.zeros(0, dt)
    return out


def _to_struct(fm: Format, keep: list) -> OrcFormat:
    s = OrcFormat()
    s.M, s.N, s.segw, s.bundle, s.num_segments = fm["M"], fm["N"], fm["segw"], fm["bundle"], \
        fm["num_segments"]
    s.G = len(fm["group_depth"])
    s.nval = len(fm["val"])
    s.nitems = len(fm["item_gbeg"])
    for name in ARRAYS:
        dt = np.float32 if name == "val" else np.int32
        a = np.ascontiguousarray(fm[name], dtype=dt)
        if a.size == 0:
            a = np.zeros(1, dt)
        keep.append(a)
        setattr(s, name, _p(a, C.c_float if name == "val" else C.c_int))
    s.scale = float(fm["scale"])
    s.fp32 = int(fm["fp32"])
    return s


class OracleError(RuntimeError):
    pass


def half_scale(val) -> np.float32:
    v = _f32(val)
    return np.float32(lib().orc_half_scale(_p(v, C.c_float), v.size))


def f32_to_f16_bits(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_array(_p(x, C.c_float), _p(out, C.c_uint16), x.size)
    return out


def round_f16(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.float32)
    lib().orc_round_f16_array(_p(x, C.c_float), _p(out, C.c_float), x.size)
    return out


def build_format(row_ptr, col, val, M, N, segw=16, fp32=False) -> Format:
    rp, ci, vv = _i32(row_ptr), _i32(col), _f32(val)
    if ci.size == 0:
        ci = np.zeros(1, np.int32); vv = np.zeros(1, np.float32)
    f = OrcFormat()
    rc = lib().orc_build(_p(rp, C.c_int), _p(ci, C.c_int), _p(vv, C.c_float), M, N, segw,
                         int(fp32), C.byref(f))
    if rc != 0:
        raise OracleError(f"orc_build failed with status {rc}")
    try:
        return _take(f)
    finally:
        lib().orc_free(C.byref(f))


def canonicalize(fm: Format) -> Format:
    keep: list = []
    s = _to_struct(fm, keep)
    rc = lib().orc_canonicalize(C.byref(s))
    if rc != 0:
        raise OracleError(f"orc_canonicalize failed with status {rc}")
    out = Format({k: v for k, v in fm.items()})
    for name in ("group_rows", "lcol", "val"):
        out[name] = keep[ARRAYS.index(name)][: len(fm[name])].copy()
    return out


def spmm_csr(row_ptr, col, val, M, B, mode=0, scale=1.0):
    """Returns (R, rowL1) in float64; mode 0 = FP32 inputs, 1 = FP16 input model."""
    rp, ci, vv, Bf = _i32(row_ptr), _i32(col), _f32(val), _f32(B)
    if ci.size == 0:
        ci = np.zeros(1, np.int32); vv = np.zeros(1, np.float32)
    O = Bf.shape[1]
    R = np.empty((M, O), np.float64)
    L1 = np.empty(M, np.float64)
    lib().orc_spmm_csr(_p(rp, C.c_int), _p(ci, C.c_int), _p(vv, C.c_float), M,
                       _p(Bf, C.c_float), O, mode, float(scale), _p(R, C.c_double),
                       _p(L1, C.c_double))
    return R, L1


def spmm_check(row_ptr, col, val, M, B, prod, mode=0, scale=1.0, C0=None, threads=None,
               norms=False):
    """The parity norm's terms for every row of a product `prod` (C, M x O float32): returns (err,
    bound) with err[r] = ||C[r] - (R[r] + C0[r])||_1 and bound[r] = rowL1[r] + ||C0[r]||_1,
    R and rowL1 those of spmm_csr (same arithmetic), computed row by row on `threads` threads
    (default: up to 16) without holding R.  norms=True returns (err, bound, ref_l1, sq_err,
    sq_ref) with, per row and C_ref = R + C0, ref_l1 = ||C_ref[r]||_1 (the stricter norm),
    sq_err = ||C[r] - C_ref[r]||_2^2 and sq_ref = ||C_ref[r]||_2^2: sqrt(sum sq_err) /
    sqrt(sum sq_ref) is the reference driver's relative L2 error (main.cpp:262-275)."""
    rp, ci, vv, Bf = _i32(row_ptr), _i32(col), _f32(val), _f32(B)
    if ci.size == 0:
        ci = np.zeros(1, np.int32); vv = np.zeros(1, np.float32)
    Cf = _f32(prod)
    O = Bf.shape[1]
    if Cf.shape != (M, O):
        raise ValueError(f"C is {Cf.shape}, expected {(M, O)}")
    C0f = None if C0 is None else _f32(C0)
    if C0f is not None and C0f.shape != (M, O):
        raise ValueError(f"C0 is {C0f.shape}, expected {(M, O)}")
    if threads is None:
        threads = max(1, min(16, os.cpu_count() or 1))
    err = np.empty(M, np.float64)
    bound = np.empty(M, np.float64)
    extra = [np.empty(M, np.float64) for _ in range(3)] if norms else []
    rc = lib().orc_spmm_check(_p(rp, C.c_int), _p(ci, C.c_int), _p(vv, C.c_float), M,
                              _p(Bf, C.c_float), Bf.size, O, mode, float(scale),
                              _p(Cf, C.c_float),
                              None if C0f is None else _p(C0f, C.c_float), threads,
                              _p(err, C.c_double), _p(bound, C.c_double),
                              *([_p(x, C.c_double) for x in extra] if norms else [None] * 3))
    if rc != 0:
        raise OracleError(f"orc_spmm_check failed with status {rc}")
    return (err, bound, *extra) if norms else (err, bound)


def spmm_format(fm: Format, B) -> np.ndarray:
    keep: list = []
    s = _to_struct(fm, keep)
    Bf = _f32(B)
    R = np.empty((fm["M"], Bf.shape[1]), np.float64)
    lib().orc_spmm_format(C.byref(s), _p(Bf, C.c_float), Bf.shape[1], _p(R, C.c_double))
    return R


def cpu_spmm_f64(row_ptr, col, val, B, r0=0, r1=None, threads=1, R=None):
    """The reference driver's CPU SpMM (main.cpp:202-207) over rows [r0, r1)."""
    rp, ci, vv, Bf = _i32(row_ptr), _i32(col), _f32(val), _f32(B)
    M = rp.size - 1
    r1 = M if r1 is None else r1
    O = Bf.shape[1]
    if R is None:
        R = np.zeros((M, O), np.float64)
    if threads <= 1:
        lib().orc_cpu_spmm_f64_rows(_p(rp, C.c_int), _p(ci, C.c_int), _p(vv, C.c_float), r0, r1,
                                    _p(Bf, C.c_float), O, _p(R, C.c_double))
    else:
        lib().orc_cpu_spmm_f64_omp(_p(rp, C.c_int), _p(ci, C.c_int), _p(vv, C.c_float), r0, r1,
                                   _p(Bf, C.c_float), O, _p(R, C.c_double), threads)
    return R


def ref_build_format(row_ptr, col, val, M, N, segw=16, fp32=False) -> Format:
    """The reference's own csr_to_vcsr_mc (oracle/_ref), CPU only."""
    rp, ci, vv = _i32(row_ptr), _i32(col), _f32(val)
    if ci.size == 0:
        ci = np.zeros(1, np.int32); vv = np.zeros(1, np.float32)
    f = OrcFormat()
    err = C.create_string_buffer(512)
    rc = ref_lib().ref_build(_p(rp, C.c_int), _p(ci, C.c_int), _p(vv, C.c_float), M, N, segw,
                             int(fp32), C.byref(f), err, 512)
    if rc != 0:
        raise OracleError(err.value.decode())
    try:
        return _take(f)
    finally:
        lib().orc_free(C.byref(f))


def ref_spmm_gpu(row_ptr, col, val, M, N, dB_ptr, O, dC_ptr, segw=32, tileK=128, fp32=False):
    """C += A.B by the reference's own kernels (oracle/_ref) on the current GPU; dB_ptr (N x O
    float32) and dC_ptr (M x O float32) are device pointers.  Synchronous."""
    rp, ci, vv = _i32(row_ptr), _i32(col), _f32(val)
    if ci.size == 0:
        ci = np.zeros(1, np.int32); vv = np.zeros(1, np.float32)
    err = C.create_string_buffer(512)
    rc = ref_lib().ref_spmm_gpu(_p(rp, C.c_int), _p(ci, C.c_int), _p(vv, C.c_float), M, N, segw,
                                int(fp32), dB_ptr, O, tileK, dC_ptr, err, 512)
    if rc != 0:
        raise OracleError(err.value.decode())


def ref_half_scale(val) -> np.float32:
    v = _f32(val)
    if v.size == 0:
        v1 = np.zeros(1, np.float32)
        return np.float32(ref_lib().ref_half_scale(_p(v1, C.c_float), 0))
    return np.float32(ref_lib().ref_half_scale(_p(v, C.c_float), v.size))


def formats_equal(a: Format, b: Format) -> list:
    """Names of the fields that differ (empty list = identical, bit for bit)."""
    bad = []
    for k in ("M", "N", "segw", "bundle", "num_segments", "fp32"):
        if a[k] != b[k]:
            bad.append(k)
    if np.float32(a["scale"]).tobytes() != np.float32(b["scale"]).tobytes():
        bad.append("scale")
    for k in ARRAYS:
        x, y = np.asarray(a[k]), np.asarray(b[k])
        if x.shape != y.shape or x.tobytes() != y.tobytes():
            bad.append(k)
    return bad


# ---- column reordering (rcm_oracle.c; include/reorder.hpp:17-108) ---------------------------
def std_sort_by_key(a, key) -> np.ndarray:
    """std::sort(a, a + n, key[x] < key[y]) with libstdc++'s steps (a copy is sorted)."""
    out = _i32(a).copy()
    k = _i32(key)
    lib().orc_std_sort_by_key(_p(out, C.c_int), len(out), _p(k, C.c_int))
    return out


def rcm_order(row_ptr, col, M: int, N: int) -> np.ndarray:
    rp, ci = _i32(row_ptr), _i32(col)
    pos = np.zeros(max(N, 1), np.int32)
    st = lib().orc_rcm_order(_p(rp, C.c_int), _p(ci, C.c_int), int(M), int(N), _p(pos, C.c_int))
    if st != 0:
        raise MemoryError("orc_rcm_order")
    return pos[:N]


def apply_column_permutation(row_ptr, col, val, M: int, N: int, position, B=None, O: int = 0):
    """Returns (col, val, B_out) after the relabelling (B_out None when B is None)."""
    rp, ci, vv, pos = _i32(row_ptr), _i32(col).copy(), _f32(val).copy(), _i32(position)
    Bi = _f32(B) if B is not None else None
    Bo = np.empty_like(Bi) if Bi is not None else None
    st = lib().orc_apply_column_permutation(
        _p(rp, C.c_int), _p(ci, C.c_int), _p(vv, C.c_float), int(M), int(N), _p(pos, C.c_int),
        _p(Bi, C.c_float) if Bi is not None else None, int(O),
        _p(Bo, C.c_float) if Bo is not None else None)
    if st != 0:
        raise MemoryError("orc_apply_column_permutation")
    return ci, vv, Bo


def heap_sort_by_key(a, key) -> np.ndarray:
    out = _i32(a).copy()
    k = _i32(key)
    lib().orc_heap_sort_by_key(_p(out, C.c_int), len(out), _p(k, C.c_int))
    return out


def ref_partial_sort_by_key(a, key) -> np.ndarray:
    out = _i32(a).copy()
    k = _i32(key)
    ref_lib().ref_partial_sort_by_key(_p(out, C.c_int), len(out), _p(k, C.c_int))
    return out


def ref_sort_adversary(n: int) -> np.ndarray:
    keys = np.zeros(max(n, 1), np.int32)
    ref_lib().ref_sort_adversary(int(n), _p(keys, C.c_int))
    return keys[:n]


def ref_std_sort_by_key(a, key) -> np.ndarray:
    out = _i32(a).copy()
    k = _i32(key)
    ref_lib().ref_std_sort_by_key(_p(out, C.c_int), len(out), _p(k, C.c_int))
    return out


def ref_rcm_order(row_ptr, col, M: int, N: int) -> np.ndarray:
    rp, ci = _i32(row_ptr), _i32(col)
    pos = np.zeros(max(N, 1), np.int32)
    ref_lib().ref_rcm_order(_p(rp, C.c_int), _p(ci, C.c_int), int(M), int(N), _p(pos, C.c_int))
    return pos[:N]


def ref_apply_column_permutation(row_ptr, col, val, M: int, N: int, position, B=None, O: int = 0):
    rp, ci, vv, pos = _i32(row_ptr), _i32(col).copy(), _f32(val).copy(), _i32(position)
    Bi = _f32(B).copy() if B is not None else None
    ref_lib().ref_apply_column_permutation(_p(rp, C.c_int), _p(ci, C.c_int), _p(vv, C.c_float),
                                           int(M), int(N), _p(pos, C.c_int),
                                           _p(Bi, C.c_float) if Bi is not None else None, int(O))
    return ci, vv, Bi
