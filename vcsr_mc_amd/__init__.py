"""vcsr_mc_amd -- MI355X (gfx950) VCSR-MC SpMM.

Python mirror of the reference's C++ surface (MuuSeoTia/VCSR_MC include/vcsr_formats.hpp:11-26)
over the C ABI of ``libvcsrmc.so`` (include/vcsrmc.h).  Device buffers are torch tensors on a
ROCm device; torch is only the allocator and stream provider here.  The compute path is the
HIP library: if it is not built, every entry point raises, there is no fallback.

Reference name                        here
------------------------------------  -----------------------------------------------
half_scale(const CSR&)                half_scale(csr)
csr_to_vcsr_mc(csr, fp32, segw)       csr_to_vcsr_mc(csr, fp32=False, segw=16)
upload_vcsr_mc_device(V)              upload_vcsr_mc_device(V)
run_vcsr_mc_spmm_gpu(V, dB, O, ...)   run_vcsr_mc_spmm_gpu(V, dB, O, tileK, dC, stream) -> ms
destroy_vcsr_mc_device(st)            destroy_vcsr_mc_device(stream)

``DeviceFormat`` is the handle-based form (several formats at once, GPU build straight from a
device CSR, FP16 B).
"""
from __future__ import annotations

import ctypes as C
import os
import weakref
from dataclasses import dataclass, field

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libvcsrmc.so")
BENCH_LIB_PATH = os.path.join(HERE, "libvcsrmc_bench.so")

OK, ERR_ARG, ERR_SEGW, ERR_TILEK, ERR_CSR, ERR_UNSORTED, ERR_FORMAT, ERR_OVERFLOW, ERR_HIP, \
    ERR_STATE, ERR_SCRATCH = range(11)
NOALLOC_SCRATCH_BYTES = 64 << 20
B_F32, B_F16 = 0, 1
SPMM_OVERWRITE = 1


class VCSRMCError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(msg)
        self.status = status


class _Info(C.Structure):
    _fields_ = [
        ("M", C.c_int), ("N", C.c_int), ("segw", C.c_int), ("bundle", C.c_int),
        ("num_segments", C.c_int), ("num_groups", C.c_int), ("nval", C.c_longlong),
        ("num_items", C.c_int), ("scale", C.c_float), ("fp32", C.c_int), ("nnz", C.c_longlong),
        ("num_panels", C.c_int), ("num_chunks", C.c_int), ("num_units", C.c_int),
        ("device", C.c_int), ("num_dense", C.c_int), ("row_grouped", C.c_int),
        ("num_heavy", C.c_int), ("num_split_panels", C.c_int),
        ("num_row_step_batches", C.c_int),
    ]


class _Traffic(C.Structure):
    _fields_ = [
        ("b_bytes", C.c_longlong), ("b_once_bytes", C.c_longlong), ("a_bytes", C.c_longlong),
        ("c_bytes", C.c_longlong), ("convert_bytes", C.c_longlong), ("total", C.c_longlong),
        ("o_tile_width", C.c_int), ("o_tiles", C.c_int), ("row_parts", C.c_int),
    ]


_lib_handle = None
_bench_handle = None


def _one_hip_runtime():
    """Loads torch's HIP runtime before either library.  torch ships its own libamdhip64
    (soname libamdhip64.so.7, needed by torch as libamdhip64.so); loaded first, it also serves
    the libraries' libamdhip64.so.7.  Loaded the other way round, the process would hold two
    HIP runtimes, and the second to open the GPU finds no device."""
    import torch  # noqa: F401


def lib():
    """The product library; raises if it has not been built."""
    global _lib_handle
    if _lib_handle is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        _one_hip_runtime()
        L = C.CDLL(LIB_PATH)
        vp, ip, fp = C.c_void_p, C.POINTER(C.c_int), C.POINTER(C.c_float)
        L.vcsrmc_create.argtypes = [C.POINTER(vp)]
        L.vcsrmc_destroy.argtypes = [vp]
        L.vcsrmc_half_scale.argtypes = [vp, C.c_longlong, fp, vp]
        L.vcsrmc_build_csr.argtypes = [vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int,
                                       C.c_int, vp]
        L.vcsrmc_upload.argtypes = [vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                    C.c_longlong, C.c_int, vp, vp, vp, vp, vp, vp, vp, vp,
                                    C.c_float, C.c_int, vp]
        L.vcsrmc_get_info.argtypes = [vp, C.POINTER(_Info)]
        L.vcsrmc_download.argtypes = [vp] + [vp] * 8
        L.vcsrmc_spmm.argtypes = [vp, vp, C.c_int, C.c_int, C.c_int, vp, vp, fp]
        L.vcsrmc_spmm_ex.argtypes = [vp, vp, C.c_int, C.c_int, C.c_int, vp, C.c_int, vp, fp]
        L.vcsrmc_spmm_noalloc.argtypes = [vp, vp, C.c_int, C.c_int, C.c_int, vp, C.c_int, vp]
        L.vcsrmc_rcm_order.argtypes = [vp, vp, C.c_int, C.c_int, C.c_int, vp, vp]
        L.vcsrmc_set_rcm_limits.argtypes = [C.c_longlong, C.c_longlong]
        L.vcsrmc_set_row_grouping.argtypes = [C.c_int]
        L.vcsrmc_set_fp32_row_steps.argtypes = [C.c_int]
        L.vcsrmc_get_row_map.argtypes = [vp, vp, C.c_longlong, C.POINTER(C.c_longlong)]
        L.vcsrmc_apply_column_permutation.argtypes = [vp, vp, vp, C.c_int, C.c_int, C.c_int, vp,
                                                      vp, C.c_int, vp, vp]
        L.vcsrmc_get_units.argtypes = [vp, vp, C.c_longlong, C.POINTER(C.c_longlong), vp]
        L.vcsrmc_traffic_floor.argtypes = [vp, C.c_int, C.c_int, C.c_int, C.c_int,
                                           C.POINTER(_Traffic), vp]
        L.vcsrmc_status_string.restype = C.c_char_p
        L.vcsrmc_status_string.argtypes = [C.c_int]
        L.vcsrmc_last_error.restype = C.c_char_p
        for f in ("vcsrmc_create", "vcsrmc_destroy", "vcsrmc_half_scale", "vcsrmc_build_csr",
                  "vcsrmc_upload", "vcsrmc_get_info", "vcsrmc_download", "vcsrmc_spmm",
                  "vcsrmc_spmm_ex", "vcsrmc_spmm_noalloc", "vcsrmc_rcm_order",
                  "vcsrmc_set_rcm_limits", "vcsrmc_set_row_grouping", "vcsrmc_get_row_map",
                  "vcsrmc_apply_column_permutation", "vcsrmc_set_fp32_row_steps",
                  "vcsrmc_get_units", "vcsrmc_traffic_floor"):
            getattr(L, f).restype = C.c_int
        _lib_handle = L
    return _lib_handle


def bench_lib():
    global _bench_handle
    if _bench_handle is None:
        if not os.path.exists(BENCH_LIB_PATH):
            raise ImportError(f"{BENCH_LIB_PATH} is not built (run __graft_entry__.build())")
        _one_hip_runtime()
        L = C.CDLL(BENCH_LIB_PATH)
        vp = C.c_void_p
        L.vcsrmc_gen.argtypes = [C.c_int, C.c_int, C.c_ulonglong, C.POINTER(vp)]
        L.vcsrmc_gen_info.argtypes = [vp, C.POINTER(C.c_int), C.POINTER(C.c_int),
                                      C.POINTER(C.c_longlong)]
        L.vcsrmc_gen_copy.argtypes = [vp, vp, vp, vp]
        L.vcsrmc_gen_free.argtypes = [vp]
        L.vcsrmc_gen_dense.argtypes = [C.c_int, C.c_ulonglong, C.c_int, vp, C.c_longlong]
        L.vcsrmc_rocsparse_spmm.argtypes = [C.c_int, C.c_int, C.c_int, vp, vp, vp, C.c_int, vp,
                                            C.c_int, C.c_int, vp, C.c_float, C.c_int, vp,
                                            C.POINTER(C.c_float), C.POINTER(C.c_float)]
        for f in ("vcsrmc_gen", "vcsrmc_gen_info", "vcsrmc_gen_copy", "vcsrmc_gen_free",
                  "vcsrmc_gen_dense", "vcsrmc_rocsparse_spmm", "vcsrmc_rocsparse_release"):
            getattr(L, f).restype = C.c_int
        _bench_handle = L
    return _bench_handle


def _check(status: int, what: str) -> None:
    if status != OK:
        detail = lib().vcsrmc_last_error().decode(errors="replace")
        raise VCSRMCError(status, f"{what}: {detail or lib().vcsrmc_status_string(status).decode()}")


def _ptr(x) -> int | None:
    """Raw address of a torch tensor or numpy array (None stays None)."""
    if x is None:
        return None
    if isinstance(x, np.ndarray):
        return x.ctypes.data
    return int(x.data_ptr())


def _need(t, dtype, n: int, name: str, exact: bool = True) -> None:
    """Host-side check of a device operand: a contiguous CUDA tensor of `dtype` holding n
    elements (at least n when not exact), so that no kernel is launched on a short buffer."""
    ok = (t is not None and t.dtype == dtype and t.is_cuda and t.is_contiguous()
          and (t.numel() == n if exact else t.numel() >= n))
    if not ok:
        raise VCSRMCError(ERR_ARG, f"{name} must be a contiguous {dtype} device tensor of "
                                   f"{'' if exact else 'at least '}{n} elements")


def _stream_ptr(stream) -> int | None:
    if stream is None:
        import torch
        return int(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, int):
        return stream
    return int(stream.cuda_stream)


# ---- host containers mirroring the reference structs -------------------------------------
@dataclass
class CSR:
    """include/csr.hpp:8-13: M, N, nnz, row_ptr[M+1], col[nnz], val[nnz] (host arrays)."""
    M: int
    N: int
    nnz: int
    row_ptr: np.ndarray
    col: np.ndarray
    val: np.ndarray

    @classmethod
    def from_arrays(cls, row_ptr, col, val, M, N):
        rp = np.ascontiguousarray(row_ptr, dtype=np.int32)
        return cls(int(M), int(N), int(rp[-1]) if len(rp) else 0, rp,
                   np.ascontiguousarray(col, dtype=np.int32),
                   np.ascontiguousarray(val, dtype=np.float32))


_FMT_ARRAYS = ("group_ptr", "group_depth", "group_seg_base", "group_rows", "lcol", "val",
               "item_gbeg", "item_gend")


@dataclass
class VCSRMC:
    """include/vcsr_formats.hpp:14-21, with numpy arrays for the std::vectors."""
    M: int = 0
    N: int = 0
    segw: int = 16
    bundle: int = 16
    num_segments: int = 0
    group_ptr: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    group_depth: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    group_seg_base: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    group_rows: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    lcol: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    val: np.ndarray = field(default_factory=lambda: np.zeros(0, np.float32))
    item_gbeg: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    item_gend: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    scale: float = 1.0
    fp32: bool = False


# ---- handle-based device format -----------------------------------------------------------
class DeviceFormat:
    """One device-resident VCSR-MC format (a vcsrmc_t handle)."""

    def __init__(self):
        h = C.c_void_p()
        _check(lib().vcsrmc_create(C.byref(h)), "vcsrmc_create")
        self._h = h
        self._mn = None  # (M, N) once a format is built or uploaded

    @property
    def handle(self):
        if self._h is None:
            raise VCSRMCError(ERR_STATE, "format closed")
        return self._h

    def close(self):
        if getattr(self, "_h", None) is not None:
            _check(lib().vcsrmc_destroy(self._h), "vcsrmc_destroy")
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @classmethod
    def from_device_csr(cls, row_ptr, col, val, M, N, fp32=False, segw=16, stream=None):
        """GPU build from torch device tensors (int32 row_ptr/col, float32 val)."""
        import torch
        nnz = int(col.numel())
        _need(row_ptr, torch.int32, int(M) + 1, "row_ptr")
        _need(col, torch.int32, nnz, "col")
        _need(val, torch.float32, nnz, "val")
        f = cls()
        _check(lib().vcsrmc_build_csr(f.handle, _ptr(row_ptr), _ptr(col) if nnz else None,
                                      _ptr(val) if nnz else None, int(M), int(N), nnz,
                                      int(bool(fp32)), int(segw), _stream_ptr(stream)),
               "vcsrmc_build_csr")
        f._mn = (int(M), int(N))
        return f

    @classmethod
    def from_host_format(cls, V: VCSRMC, stream=None):
        """Uploads caller-held format arrays.  Their lengths are checked against the sizes they
        imply (G = len(group_depth), nval = len(val), items = len(item_gbeg)) before anything
        is copied: the C ABI reads exactly those sizes from each pointer."""
        arrs = {}
        for name in _FMT_ARRAYS:
            dt = np.float32 if name == "val" else np.int32
            a = np.ascontiguousarray(getattr(V, name), dtype=dt)
            arrs[name] = a
        G = len(arrs["group_depth"])
        nval, ni = len(arrs["val"]), len(arrs["item_gbeg"])
        want = {"group_ptr": G + 1, "group_seg_base": G, "group_rows": 16 * G, "lcol": nval,
                "item_gend": ni}
        for name, n in want.items():
            if len(arrs[name]) != n:
                raise VCSRMCError(ERR_FORMAT, f"{name} holds {len(arrs[name])} entries; the "
                                              f"format's sizes need {n}")
        f = cls()
        _check(lib().vcsrmc_upload(
            f.handle, int(V.M), int(V.N), int(V.segw), int(V.bundle), int(V.num_segments), G,
            nval, ni,
            *[(arrs[n].ctypes.data if arrs[n].size else None) for n in _FMT_ARRAYS],
            float(V.scale), int(bool(V.fp32)), _stream_ptr(stream)), "vcsrmc_upload")
        return f

    def info(self) -> dict:
        i = _Info()
        _check(lib().vcsrmc_get_info(self.handle, C.byref(i)), "vcsrmc_get_info")
        return {k: getattr(i, k) for k, _ in _Info._fields_}

    def row_map(self):
        """The execution layout's row order: an int32 array, row_map[p] = the row at position p
        (-1 for padding), or None when the layout keeps natural order."""
        n = C.c_longlong(0)
        _check(lib().vcsrmc_get_row_map(self.handle, None, 0, C.byref(n)), "vcsrmc_get_row_map")
        if n.value == 0:
            return None
        out = np.zeros(n.value, np.int32)
        _check(lib().vcsrmc_get_row_map(self.handle, out.ctypes.data, out.size, C.byref(n)),
               "vcsrmc_get_row_map")
        return out

    def units(self):
        """The execution layout's work units: (units, xcd_start), units an int32 array of shape
        (num_units, 4) = {first row-order position, first tile, end tile, row mask | flags}
        (flags: 1 << 16 split panel, 1 << 17 its first unit, 1 << 18 FP32 row steps), and
        xcd_start (9 ints) the light units' XCD ranges."""
        n = C.c_longlong(0)
        xs = np.zeros(9, np.int32)
        _check(lib().vcsrmc_get_units(self.handle, None, 0, C.byref(n), xs.ctypes.data),
               "vcsrmc_get_units")
        out = np.zeros((n.value, 4), np.int32)
        if n.value:
            _check(lib().vcsrmc_get_units(self.handle, out.ctypes.data, out.size, C.byref(n),
                                          None), "vcsrmc_get_units")
        return out, xs

    def rows_of_units(self, units):
        """The C rows each unit writes, as a list of int arrays (row map applied)."""
        rmap = self.row_map()
        out = []
        for p0, _, _, w in units:
            pos = p0 + np.nonzero((int(w) >> np.arange(16)) & 1)[0]
            out.append(rmap[pos] if rmap is not None else pos)
        return out

    def traffic_floor(self, O, tileK=128, b_f16=False, overwrite=False, stream=None) -> dict:
        """HBM bytes a launch with these arguments cannot avoid under its schedule (see
        vcsrmc_traffic_floor in include/vcsrmc.h)."""
        t = _Traffic()
        _check(lib().vcsrmc_traffic_floor(self.handle, B_F16 if b_f16 else B_F32, int(O),
                                          int(tileK), SPMM_OVERWRITE if overwrite else 0,
                                          C.byref(t), _stream_ptr(stream)),
               "vcsrmc_traffic_floor")
        return {k: getattr(t, k) for k, _ in _Traffic._fields_}

    def download(self) -> VCSRMC:
        i = self.info()
        G, nval, ni = i["num_groups"], i["nval"], i["num_items"]
        out = {
            "group_ptr": np.zeros(G + 1, np.int32), "group_depth": np.zeros(G, np.int32),
            "group_seg_base": np.zeros(G, np.int32), "group_rows": np.zeros(16 * G, np.int32),
            "lcol": np.zeros(nval, np.int32), "val": np.zeros(nval, np.float32),
            "item_gbeg": np.zeros(ni, np.int32), "item_gend": np.zeros(ni, np.int32),
        }
        _check(lib().vcsrmc_download(self.handle, *[(out[n].ctypes.data if out[n].size else None)
                                                    for n in _FMT_ARRAYS]), "vcsrmc_download")
        return VCSRMC(M=i["M"], N=i["N"], segw=i["segw"], bundle=i["bundle"],
                      num_segments=i["num_segments"], scale=float(np.float32(i["scale"])),
                      fp32=bool(i["fp32"]), **out)

    def _operands(self, B, C_out, O):
        """Checks B and C_out for a multiply of width O (None: B's); returns (B dtype code, O)."""
        import torch
        b_dtype = B_F16 if B.dtype == torch.float16 else B_F32
        if B.dtype not in (torch.float16, torch.float32) or C_out.dtype != torch.float32:
            raise VCSRMCError(ERR_ARG, "B must be float16/float32 and C float32")
        if not (B.is_contiguous() and C_out.is_contiguous()):
            raise VCSRMCError(ERR_ARG, "B and C must be contiguous row-major")
        O = int(B.shape[1]) if O is None else int(O)
        if self._mn is None:
            i = self.info()
            self._mn = (i["M"], i["N"])
        M, N = self._mn
        if not (B.is_cuda and C_out.is_cuda and B.device == C_out.device):
            raise VCSRMCError(ERR_ARG, "B and C must be tensors on the same GPU")
        if O < 0 or B.numel() < N * O or C_out.numel() < M * O:
            raise VCSRMCError(ERR_ARG, f"B needs N x O = {N} x {O} and C M x O = {M} x {O} "
                                       f"elements; got {B.numel()} and {C_out.numel()}")
        return b_dtype, O

    def launcher(self, B, C_out, tileK=128, O=None, stream=None, overwrite=False):
        """A callable with no arguments that enqueues spmm(B, C_out, ...) asynchronously, with
        the checks and the ctypes conversions done once here: for loops of launches whose
        kernels are shorter than the checks (a 6 us multiply).  It holds this format, B and
        C_out; once the format is closed, calling it raises ERR_STATE."""
        b_dtype, O = self._operands(B, C_out, O)
        fn = lib().vcsrmc_spmm_ex
        h = self.handle
        args = (h, C.c_void_p(_ptr(B)), C.c_int(b_dtype), C.c_int(O),
                C.c_int(int(tileK)), C.c_void_p(_ptr(C_out)),
                C.c_int(SPMM_OVERWRITE if overwrite else 0), C.c_void_p(_stream_ptr(stream)),
                None)
        keep = (self, B, C_out)

        def launch():
            if keep[0]._h is not h:
                raise VCSRMCError(ERR_STATE, "format closed")
            rc = fn(*args)
            if rc != 0:
                _check(rc, "vcsrmc_spmm")

        return launch

    def spmm(self, B, C_out, tileK=128, O=None, stream=None, timed=False, overwrite=False):
        """C_out += A . B on the GPU (overwrite: C_out = A . B on the rows A touches, C_out
        not read).  B: (N, O) float32 or float16 device tensor; C_out: (M, O) float32.
        Returns the event-timed kernel time in ms when timed, else None."""
        b_dtype, O = self._operands(B, C_out, O)
        ms = C.c_float(0.0)
        _check(lib().vcsrmc_spmm_ex(self.handle, _ptr(B), b_dtype, O, int(tileK), _ptr(C_out),
                                    SPMM_OVERWRITE if overwrite else 0, _stream_ptr(stream),
                                    C.byref(ms) if timed else None),
               "vcsrmc_spmm")
        return ms.value if timed else None


# ---- the reference's free functions (global single format, src/vcsr_mc.cu:126-131) ---------
_global = {"fmt": None, "uploaded": False}


def half_scale(csr: CSR) -> float:
    import torch
    v = torch.from_numpy(np.ascontiguousarray(csr.val, np.float32)).cuda()
    s = C.c_float(1.0)
    _check(lib().vcsrmc_half_scale(_ptr(v) if v.numel() else None, int(v.numel()), C.byref(s),
                                   _stream_ptr(None)), "half_scale")
    return s.value


def csr_to_vcsr_mc(csr: CSR, fp32: bool = False, segw: int = 16) -> VCSRMC:
    """The format, built on the GPU and copied back (include/vcsr_formats.hpp:22)."""
    import torch
    if segw not in (16, 32, 48, 64):
        raise VCSRMCError(ERR_SEGW, "vcsr_mc supports segw in {16, 32, 48, 64}")
    rp = torch.from_numpy(np.ascontiguousarray(csr.row_ptr, np.int32)).cuda()
    ci = torch.from_numpy(np.ascontiguousarray(csr.col, np.int32)).cuda()
    vv = torch.from_numpy(np.ascontiguousarray(csr.val, np.float32)).cuda()
    with DeviceFormat.from_device_csr(rp, ci, vv, csr.M, csr.N, fp32, segw) as f:
        return f.download()


def upload_vcsr_mc_device(V: VCSRMC) -> None:
    if _global["uploaded"]:
        return
    _global["fmt"] = DeviceFormat.from_host_format(V)
    _global["uploaded"] = True


def run_vcsr_mc_spmm_gpu(V: VCSRMC, dB, O: int, tileK: int, dC, stream=None) -> float:
    """C += A . B, event-timed like the reference (returns ms)."""
    if len(V.item_gbeg) == 0:
        return 0.0
    if not _global["uploaded"]:
        upload_vcsr_mc_device(V)
    return _global["fmt"].spmm(dB, dC, tileK=tileK, O=O, stream=stream, timed=True)


def destroy_vcsr_mc_device(stream=None) -> None:
    if _global["fmt"] is not None:
        _global["fmt"].close()
    _global["fmt"] = None
    _global["uploaded"] = False


# ---- execution layout ----------------------------------------------------------------------
ROW_GROUPING_OFF, ROW_GROUPING_AUTO, ROW_GROUPING_ALWAYS = 0, 1, 2


def set_row_grouping(mode: int) -> None:
    """Row order of the execution layout for later builds (process-wide): ROW_GROUPING_OFF
    (natural order), ROW_GROUPING_AUTO (the default: rows grouped by shared columns where that
    saves tiles) or ROW_GROUPING_ALWAYS.  DeviceFormat.info()["row_grouped"] tells which a
    format holds."""
    _check(lib().vcsrmc_set_row_grouping(int(mode)), "set_row_grouping")


FP32_ROW_STEPS_OFF, FP32_ROW_STEPS_AUTO, FP32_ROW_STEPS_ALWAYS = 0, 1, 2


def set_fp32_row_steps(mode: int) -> None:
    """Product of FP32 panels for later builds (process-wide): FP32_ROW_STEPS_OFF (tiles of
    16 x 16 x 4 matrix-core steps only), FP32_ROW_STEPS_AUTO (the default: panels whose rows
    rarely share a column run row steps of v_mfma_f32_4x4x1_16b_f32) or FP32_ROW_STEPS_ALWAYS.
    DeviceFormat.info()["num_row_step_batches"] tells how many batches a format holds."""
    _check(lib().vcsrmc_set_fp32_row_steps(int(mode)), "set_fp32_row_steps")


# ---- column reordering (include/reorder.hpp:17-108), computed on the GPU -------------------
def rcm_order_device(row_ptr, col, M: int, N: int, position, stream=None) -> None:
    """Device tensors: position[N] (int32) = new position of every old column."""
    import torch
    nnz = int(col.numel())
    _need(row_ptr, torch.int32, int(M) + 1, "row_ptr")
    _need(col, torch.int32, nnz, "col")
    _need(position, torch.int32, int(N), "position", exact=False)
    _check(lib().vcsrmc_rcm_order(_ptr(row_ptr), _ptr(col) if nnz else None, int(M), int(N), nnz,
                                  _ptr(position) if N else None, _stream_ptr(stream)),
           "rcm_column_order")


def apply_column_permutation_device(row_ptr, col, val, M: int, N: int, position, B=None,
                                    B_out=None, O: int = 0, stream=None) -> None:
    """Device tensors; col and val relabelled in place, B_out[position[r]] = B[r]."""
    import torch
    nnz = int(col.numel())
    _need(row_ptr, torch.int32, int(M) + 1, "row_ptr")
    _need(col, torch.int32, nnz, "col")
    _need(val, torch.float32, nnz, "val")
    _need(position, torch.int32, int(N), "position", exact=False)
    if B is not None:
        _need(B, torch.float32, int(N) * int(O), "B", exact=False)
        _need(B_out, torch.float32, int(N) * int(O), "B_out", exact=False)
    _check(lib().vcsrmc_apply_column_permutation(
        _ptr(row_ptr), _ptr(col) if nnz else None, _ptr(val) if nnz else None, int(M), int(N),
        nnz, _ptr(position) if N else None, _ptr(B), int(O), _ptr(B_out), _stream_ptr(stream)),
        "apply_column_permutation")


def rcm_column_order(csr: CSR) -> np.ndarray:
    """new_position[old_column] of the reverse Cuthill-McKee order (reorder.hpp:17-77)."""
    import torch
    rp = torch.from_numpy(np.ascontiguousarray(csr.row_ptr, np.int32)).cuda()
    ci = torch.from_numpy(np.ascontiguousarray(csr.col, np.int32)).cuda()
    pos = torch.empty(max(csr.N, 1), dtype=torch.int32, device="cuda")
    rcm_order_device(rp, ci, csr.M, csr.N, pos)
    return pos[:csr.N].cpu().numpy()


def apply_column_permutation(csr: CSR, hB, O: int, position) -> tuple[CSR, np.ndarray | None]:
    """(A P, P^T B) of reorder.hpp:82-108; returns the new CSR and B (None if hB is None)."""
    import torch
    rp = torch.from_numpy(np.ascontiguousarray(csr.row_ptr, np.int32)).cuda()
    ci = torch.from_numpy(np.ascontiguousarray(csr.col, np.int32)).cuda()
    vv = torch.from_numpy(np.ascontiguousarray(csr.val, np.float32)).cuda()
    pos = torch.from_numpy(np.ascontiguousarray(position, np.int32)).cuda()
    B = Bo = None
    if hB is not None:
        B = torch.from_numpy(np.ascontiguousarray(hB, np.float32).reshape(-1)).cuda()
        Bo = torch.empty_like(B)
    apply_column_permutation_device(rp, ci, vv, csr.M, csr.N, pos, B, Bo, O)
    out = CSR(csr.M, csr.N, csr.nnz, np.array(csr.row_ptr, np.int32), ci.cpu().numpy(),
              vv.cpu().numpy())
    return out, (Bo.cpu().numpy().reshape(np.shape(hB)) if hB is not None else None)


# ---- workloads (libvcsrmc_bench.so) --------------------------------------------------------
SEED_BASE = 20260923  # the reference's fixed seed (src/main.cpp:165); workload k uses +k

WORKLOADS = {
    1: dict(name="uniform", precision="fp32", O=128),
    2: dict(name="powerlaw", precision="fp16", O=128),
    3: dict(name="stencil27", precision="fp32", O=128),
    4: dict(name="block32", precision="fp16", O=256),
    5: dict(name="rmat", precision="fp16", O=128),
}


def generate(config: int, size: int = 0, seed: int | None = None) -> CSR:
    """Seeded synthetic matrix of a benchmark workload (see include/vcsrmc_bench.h)."""
    L = bench_lib()
    seed = SEED_BASE + config if seed is None else seed
    h = C.c_void_p()
    if L.vcsrmc_gen(int(config), int(size), C.c_ulonglong(seed), C.byref(h)) != 0:
        raise VCSRMCError(ERR_ARG, f"generator failed for config {config} size {size}")
    try:
        M, N, nnz = C.c_int(), C.c_int(), C.c_longlong()
        L.vcsrmc_gen_info(h, C.byref(M), C.byref(N), C.byref(nnz))
        rp = np.empty(M.value + 1, np.int32)
        col = np.empty(nnz.value, np.int32)
        val = np.empty(nnz.value, np.float32)
        L.vcsrmc_gen_copy(h, rp.ctypes.data, col.ctypes.data if nnz.value else None,
                          val.ctypes.data if nnz.value else None)
    finally:
        L.vcsrmc_gen_free(h)
    return CSR(M.value, N.value, nnz.value, rp, col, val)


def dense(n_rows: int, n_cols: int, seed: int, dist: int = 0, fp16_exact: bool = False) -> np.ndarray:
    out = np.empty((n_rows, n_cols), np.float32)
    if bench_lib().vcsrmc_gen_dense(int(dist), C.c_ulonglong(seed), int(fp16_exact),
                                    out.ctypes.data, out.size) != 0:
        raise VCSRMCError(ERR_ARG, "dense generator failed")
    return out


# The A operand of the hipSPARSE plans the bench library keeps: weak references to the tensors
# and their version counters.  The library keys plans by device address, so a new matrix at a
# reused address would find another matrix's analysis; the session is released first whenever
# A is not the same live tensors, unmodified.
_rs_matrix = None


def _rs_same_matrix(tensors) -> bool:
    global _rs_matrix
    now = [(weakref.ref(t), t._version) for t in tensors]
    same = _rs_matrix is not None and all(r() is t and v == t._version
                                          for (r, v), t in zip(_rs_matrix, tensors))
    _rs_matrix = now
    return same


def rocsparse_spmm(M, N, row_ptr, col, val, B, C_out, alpha=1.0, alg=0, stream=None):
    """hipSPARSE SpMM C = alpha A.B (beta 0) on device tensors; returns (ms, setup_ms).  Plans
    (descriptors, buffer, preprocess analysis) are kept while A is the same tensors."""
    import torch
    if not _rs_same_matrix((row_ptr, col, val)):
        bench_lib().vcsrmc_rocsparse_release()
    ms, setup = C.c_float(0.0), C.c_float(0.0)
    rc = bench_lib().vcsrmc_rocsparse_spmm(
        int(M), int(N), int(col.numel()), _ptr(row_ptr), _ptr(col), _ptr(val),
        int(val.dtype == torch.float16), _ptr(B), int(B.dtype == torch.float16), int(B.shape[1]),
        _ptr(C_out), float(alpha), int(alg), _stream_ptr(stream), C.byref(ms), C.byref(setup))
    if rc != 0:
        raise VCSRMCError(ERR_HIP, f"hipSPARSE SpMM failed ({rc})")
    return ms.value, setup.value
