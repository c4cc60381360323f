"""ctypes loader of the MI355X fitter library, API of cusr/kernel/co_inproc.py.

`InProcessCO(device_id, lib_path, variant).optimize(pop, max_iter)` and the
process-wide `get_inproc_co(device_id, variant)` keep the reference's names,
arguments, return dicts and `COError` codes (co_inproc.py:51-57,101-295): a pop
dict (popio keys M, total_nodes, ..., nt, nv, ci, metas, c_init, xs, ym) goes
in; {'c_final', 'status', 'loss_init', 'loss_final'} (fp32) comes out.

Extensions with no reference counterpart:
  optimize_ex(pop, ...)  fp64 constants/data/outputs, AD mode and precision
  evaluate(pop, c)       y[m, i] = f_m(x_i; c_m) on the device
  decode(pop)            host-only checks, device programs and K bins

There is no CPU path: when the library is not built these raise.
"""
from __future__ import annotations

import atexit
import ctypes
import os
import threading
from pathlib import Path

import numpy as np

POP_MAGIC = 0x4D4C344D
POP_VERSION = 1

CO_OK = 0
CO_ERR_BOUNDS = 2
CO_ERR_CUDA = -1
CO_ERR_SUM_C = -2
CO_ERR_SUM_NODES = -3
CO_ERR_NULLARG = -4
CO_ERR_OOM = -5
CO_ERR_PROGRAM = -6
CO_ERR_DATA = -7

# bounds (include/cusr_co.h): K and value stack as the reference's
# (cusr/kernel/ad_interp.cuh:34-39), variables up to 255, any number of nodes
CO_MAX_K = 32
CO_MAX_STACK = 64
CO_MAX_VARS = 255
# the fast kernels' share (co_fast_path); the general kernel fits the rest
CO_FAST_MAX_K, CO_FAST_MAX_STACK, CO_FAST_MAX_VARS, CO_FAST_MAX_NODES = 16, 16, 8, 255
CO_GENERAL_BIN = CO_FAST_MAX_K + 1
CO_BINS = CO_FAST_MAX_K + 2
# point partitions (include/cusr_co.h co_partitions_for_n): beyond
# CO_MAX_PARTITIONS each partition is a workgroup (the split path)
CO_MAX_PARTITIONS, CO_MAX_SPLIT, CO_SPLIT_MIN_N = 4, 256, 65536
CO_STATIC_SCRATCH_BYTES = 64 << 20


def co_partitions_for_n(N: int) -> int:
    """include/cusr_co.h co_partitions_for_n."""
    if N >= CO_SPLIT_MIN_N:
        g = 8
        while g < CO_MAX_SPLIT and g * 2 * 4096 <= N:
            g *= 2
        return g
    return 4 if N >= 16384 else (2 if N >= 512 else 1)


def co_partitions_for(N: int, ad_mode: int = 0) -> int:
    """include/cusr_co.h co_partitions_for: reverse AD from 2,048 to 16,383
    points takes the split path with 8 partitions."""
    if ad_mode == 1 and 2048 <= N < 16384:
        return 8
    return co_partitions_for_n(N)

CO_AD_FORWARD, CO_AD_REVERSE = 0, 1
CO_PREC_FP64, CO_PREC_MIXED = 0, 1
CO_ORDER_IMPROVE_FIRST, CO_ORDER_CONVERGE_FIRST = 0, 1
# damped-solve variants (cusr_co.h CoOptions.damping; cusr/kernel/batch_lm_ad.cu:149-172)
CO_DAMP_RELATIVE, CO_DAMP_TRUST_REGION, CO_DAMP_PIVOT_FLOOR = 0, 1, 2
CO_PIVOT_FLOOR_EPS = float(np.float32(1e-9))          # the reference's 1e-9f
CO_TRUST_REGION_LAMBDA0 = float(np.float32(1e-4))     # its trust-region start
POP_FLAG_F64, POP_FLAG_SHARED_Y = 1, 2
# external statuses (include/pop_format.h, cusr/kernel/lm_core.cuh:46-56)
STATUS_CONVERGED, STATUS_MAXITER, STATUS_FAIL_NAN, STATUS_K0_SKIP, STATUS_FAIL_CHOLESKY = 0, 1, 2, 3, 4

_ERR_MSG = {
    CO_ERR_BOUNDS: (f"beyond device bounds (K<={CO_MAX_K}, max_stack<={CO_MAX_STACK}, "
                    f"n_vars<={CO_MAX_VARS}), or LDS rows beyond the device's LDS"),
    CO_ERR_CUDA: "HIP error inside the library",
    CO_ERR_SUM_C: "sum(metas.K) != header.total_c (pop inconsistent)",
    CO_ERR_SUM_NODES: "sum(metas.n_nodes) != header.total_nodes (pop inconsistent)",
    CO_ERR_NULLARG: "null pointer / bad argument",
    CO_ERR_OOM: "out of memory growing a device buffer",
    CO_ERR_PROGRAM: "malformed expression (unknown op, bad node, rank or variable index)",
    CO_ERR_DATA: "no data set uploaded, or the population's N / n_vars differ from it",
}


class COError(RuntimeError):
    """A non-OK return code of the library (co_inproc.py:51-57)."""

    def __init__(self, code: int, where: str):
        self.code = code
        super().__init__(f"{where}: {_ERR_MSG.get(code, f'unknown code {code}')} (code={code})")


class PopHeader(ctypes.Structure):
    """pop_format.h PopHeader: 16 x int32 = 64 B."""
    _fields_ = [("magic", ctypes.c_int32), ("version", ctypes.c_int32),
                ("M_prob", ctypes.c_int32), ("total_nodes", ctypes.c_int32),
                ("total_c", ctypes.c_int32), ("N", ctypes.c_int32),
                ("n_vars", ctypes.c_int32), ("K_max", ctypes.c_int32),
                ("max_stack", ctypes.c_int32), ("reserved", ctypes.c_int32 * 7)]


class TreeMeta(ctypes.Structure):
    """pop_format.h TreeMeta: 4 x int32 = 16 B."""
    _fields_ = [("node_offset", ctypes.c_int32), ("n_nodes", ctypes.c_int32),
                ("c_offset", ctypes.c_int32), ("K", ctypes.c_int32)]


class CoOptions(ctypes.Structure):
    """cusr_co.h CoOptions."""
    _fields_ = [("struct_size", ctypes.c_int32), ("ad_mode", ctypes.c_int32),
                ("precision", ctypes.c_int32), ("max_iter", ctypes.c_int32),
                ("lambda0", ctypes.c_double), ("xtol", ctypes.c_double),
                ("fp64_guard", ctypes.c_int32), ("partitions", ctypes.c_int32),
                ("lm_order", ctypes.c_int32), ("tail_iter", ctypes.c_int32),
                ("tail_partitions", ctypes.c_int32), ("f32_range", ctypes.c_int32),
                ("damping", ctypes.c_int32), ("reserved", ctypes.c_int32)]


assert ctypes.sizeof(PopHeader) == 64
assert ctypes.sizeof(TreeMeta) == 16
assert ctypes.sizeof(CoOptions) == 64

_VP = ctypes.c_void_p
_HERE = Path(__file__).resolve().parent

# every extern "C" symbol of include/cusr_co.h
EXPORTED = ("co_init", "co_optimize", "co_last_split", "co_teardown", "co_options_default",
            "co_optimize_ex", "co_eval_ex", "co_upload_ex", "co_fit_resident",
            "co_last_kernel_ms", "co_last_bin_ms", "co_decode", "co_data_upload",
            "co_optimize_data", "co_data_upload_device", "co_optimize_data_device",
            "co_narrow_fp32",
            "co_fit_resident_static")


def lib_path(variant: str = "ad") -> Path:
    """libcusr_co_<variant>.so next to this module (cusr_amd/build.py output)."""
    return _HERE / f"libcusr_co_{variant}.so"


def _arr(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a, a.ctypes.data_as(_VP)


def _header(pop: dict) -> PopHeader:
    """Full 64-B header from a pop dict (co_inproc.py:148-163)."""
    h = PopHeader()
    h.magic, h.version = POP_MAGIC, POP_VERSION
    h.M_prob = int(pop["M"])
    h.total_nodes = int(pop["total_nodes"])
    h.total_c = int(pop["total_c"])
    h.N = int(pop["N"])
    h.n_vars = int(pop["n_vars"])
    h.K_max = int(pop["K_max"])
    h.max_stack = int(pop["max_stack"])
    if pop.get("shared_y"):
        # pop.bin v2: ym is one row [N] shared by every expression
        h.version = 2
        h.reserved[0] = POP_FLAG_SHARED_Y
    return h


def _sized(a, dtype, count: int, name: str):
    """_arr with the element count the header implies; a short host array
    would be read past its end by the library's copy."""
    a, p = _arr(a, dtype)
    if a.size != count:
        raise ValueError(f"{name} has {a.size} elements, the header implies {count}")
    return a, p


def _counts(pop: dict):
    """(c_init, xs, ym) element counts of a pop dict (ym is one row when the
    target is shared)."""
    M, N = int(pop["M"]), int(pop["N"])
    rows = 1 if pop.get("shared_y") else M
    return int(pop["total_c"]), N * int(pop["n_vars"]), rows * N


def _metas(pop: dict):
    M = int(pop["M"])
    m = np.ascontiguousarray(pop["metas"], dtype=np.int32).reshape(M, 4)
    return m, m.ctypes.data_as(_VP)


def _bind(lib) -> None:
    i32, dbl = ctypes.c_int32, ctypes.c_double
    lib.co_init.argtypes = [ctypes.c_int, ctypes.POINTER(_VP)]
    lib.co_init.restype = ctypes.c_int
    lib.co_optimize.argtypes = [_VP, ctypes.POINTER(PopHeader)] + [_VP] * 7 + [ctypes.c_int] + [_VP] * 4
    lib.co_optimize.restype = ctypes.c_int
    lib.co_optimize_ex.argtypes = [_VP, ctypes.POINTER(CoOptions), ctypes.POINTER(PopHeader)] + [_VP] * 12
    lib.co_optimize_ex.restype = ctypes.c_int
    lib.co_eval_ex.argtypes = [_VP, ctypes.POINTER(PopHeader)] + [_VP] * 6 + [ctypes.c_int, _VP]
    lib.co_eval_ex.restype = ctypes.c_int
    lib.co_upload_ex.argtypes = [_VP, ctypes.POINTER(PopHeader)] + [_VP] * 7
    lib.co_upload_ex.restype = ctypes.c_int
    lib.co_fit_resident.argtypes = [_VP, ctypes.POINTER(CoOptions)] + [_VP] * 5
    lib.co_fit_resident.restype = ctypes.c_int
    lib.co_fit_resident_static.argtypes = [_VP, ctypes.POINTER(CoOptions)] + [_VP] * 5
    lib.co_fit_resident_static.restype = ctypes.c_int
    lib.co_data_upload.argtypes = [_VP, ctypes.c_int, ctypes.c_int, _VP, _VP]
    lib.co_data_upload.restype = ctypes.c_int
    lib.co_data_upload_device.argtypes = [_VP, ctypes.c_int, ctypes.c_int, _VP, _VP]
    lib.co_data_upload_device.restype = ctypes.c_int
    lib.co_optimize_data.argtypes = [_VP, ctypes.POINTER(CoOptions), ctypes.POINTER(PopHeader)] + [_VP] * 10
    lib.co_optimize_data.restype = ctypes.c_int
    lib.co_optimize_data_device.argtypes = ([_VP, ctypes.POINTER(CoOptions),
                                             ctypes.POINTER(PopHeader)] + [_VP] * 10)
    lib.co_optimize_data_device.restype = ctypes.c_int
    lib.co_last_kernel_ms.argtypes = [_VP, ctypes.POINTER(dbl)]
    lib.co_last_kernel_ms.restype = ctypes.c_int
    lib.co_last_bin_ms.argtypes = [_VP, ctypes.POINTER(dbl)]
    lib.co_last_bin_ms.restype = ctypes.c_int
    lib.co_decode.argtypes = [ctypes.POINTER(PopHeader)] + [_VP] * 10
    lib.co_decode.restype = ctypes.c_int
    lib.co_narrow_fp32.argtypes = [ctypes.POINTER(PopHeader)] + [_VP] * 9
    lib.co_narrow_fp32.restype = ctypes.c_int
    lib.co_last_split.argtypes = [ctypes.POINTER(dbl), ctypes.POINTER(dbl)]
    lib.co_last_split.restype = ctypes.c_int
    lib.co_teardown.argtypes = [_VP]
    lib.co_teardown.restype = None
    lib.co_options_default.argtypes = [ctypes.POINTER(CoOptions)]
    lib.co_options_default.restype = None
    del i32


_LIBS: dict[str, ctypes.CDLL] = {}


def load_library(variant: str = "ad", path: str | Path | None = None) -> ctypes.CDLL:
    """dlopen the built library (no device call). Raises if it is not built.
    CUSR_CO_LIB in the environment names another build of the same library."""
    if path is None and os.environ.get("CUSR_CO_LIB"):
        path = os.environ["CUSR_CO_LIB"]
    p = Path(path) if path is not None else lib_path(variant)
    key = str(p.resolve()) if p.exists() else str(p)
    if key not in _LIBS:
        if not p.exists():
            raise FileNotFoundError(f"{p} is not built: run `python -m cusr_amd.build`")
        lib = ctypes.CDLL(str(p.resolve()))
        _bind(lib)
        _LIBS[key] = lib
    return _LIBS[key]


def co_fast_path(K: int, stack_depth: int, n_nodes: int, n_vars: int) -> bool:
    """include/cusr_co.h co_fast_path: the fast kernels take the expression."""
    return (K <= CO_FAST_MAX_K and stack_depth <= CO_FAST_MAX_STACK
            and n_nodes <= CO_FAST_MAX_NODES and n_vars <= CO_FAST_MAX_VARS)


def decode(pop: dict, variant: str = "ad", full: bool = False):
    """Host-only decode: (rc, program uint64[2T], order int32[M], bin_start
    int32[CO_MAX_K+2], stack int32[M]); with full, also program_off int32[M]
    (first word of each program) and route int32[M] (1: general kernel, two
    words per instruction). Needs no GPU."""
    lib = load_library(variant)
    h = _header(pop)
    T, M = int(pop["total_nodes"]), int(pop["M"])
    nt, pnt = _arr(pop["nt"], np.int32)
    nv, pnv = _arr(pop["nv"], np.float32)
    ci, pci = _arr(pop["ci"], np.int32)
    me, pme = _metas(pop)
    prog = np.zeros(max(2 * T, 1), np.uint64)
    order = np.zeros(max(M, 1), np.int32)
    bins = np.zeros(CO_MAX_K + 2, np.int32)
    stack = np.zeros(max(M, 1), np.int32)
    poff = np.zeros(max(M, 1), np.int32)
    route = np.zeros(max(M, 1), np.int32)
    rc = lib.co_decode(ctypes.byref(h), pnt, pnv, pci, pme, prog.ctypes.data_as(_VP),
                       order.ctypes.data_as(_VP), bins.ctypes.data_as(_VP),
                       stack.ctypes.data_as(_VP), poff.ctypes.data_as(_VP),
                       route.ctypes.data_as(_VP))
    out = (rc, prog[:2 * T], order[:M], bins, stack[:M])
    return out + (poff[:M], route[:M]) if full else out


def narrow_fp32(pop: dict, fit: dict, variant: str = "ad") -> dict:
    """The fp32 carrier of co_optimize applied to an fp64 fit's results
    (co_narrow_fp32, host only): {'c_final', 'status', 'loss_init',
    'loss_final', 'demoted'}; an expression whose finite fp64 constants or loss
    overflow fp32 gets its c_init back and CONVERGED becomes MAXITER."""
    lib = load_library(variant)
    h = _header(pop)
    M, C = int(pop["M"]), int(pop["total_c"])
    me, pme = _metas(pop)
    c0, pc0 = _sized(pop["c_init"], np.float64, C, "c_init")
    cf, pcf = _sized(fit["c_final"], np.float64, C, "c_final")
    li, pli = _sized(fit["loss_init"], np.float64, M, "loss_init")
    lf, plf = _sized(fit["loss_final"], np.float64, M, "loss_final")
    st = np.array(fit["status"], np.int32, copy=True)
    c32 = np.zeros(max(C, 1), np.float32)
    li32 = np.zeros(max(M, 1), np.float32)
    lf32 = np.zeros(max(M, 1), np.float32)
    rc = lib.co_narrow_fp32(ctypes.byref(h), pme, pc0, pcf, pli, plf, st.ctypes.data_as(_VP),
                            c32.ctypes.data_as(_VP), li32.ctypes.data_as(_VP),
                            lf32.ctypes.data_as(_VP))
    if rc < 0:
        raise COError(rc, "co_narrow_fp32")
    return {"c_final": c32[:C], "status": st, "loss_init": li32[:M], "loss_final": lf32[:M],
            "demoted": rc}


def default_options(**kw) -> CoOptions:
    o = CoOptions()
    o.struct_size = ctypes.sizeof(CoOptions)
    o.ad_mode, o.precision, o.max_iter = CO_AD_FORWARD, CO_PREC_FP64, 50
    o.lambda0, o.xtol, o.fp64_guard = 1e-3, 1e-6, 1
    for k, v in kw.items():
        setattr(o, k, v)
    return o


class InProcessCO:
    """One persistent device context over the library (co_inproc.py:101-246)."""

    def __init__(self, device_id: int = 0, lib_path: str | Path | None = None,
                 variant: str = "ad"):
        self.variant = variant
        self.device_id = int(device_id)
        self._lib = load_library(variant, lib_path)
        o = CoOptions()
        self._lib.co_options_default(ctypes.byref(o))
        self.default_order = int(o.lm_order)   # the library's LM ordering (ad / fd)
        self._handle = _VP()
        self._torn = False
        self._resident = (0, 0)
        self._data = None        # host copy of the uploaded data set (xs, y)
        # calls on one handle are not thread-safe (the library's buffers are
        # per handle); callers that pair upload_data with optimize_data from
        # several threads hold this across the pair
        self.lock = threading.RLock()
        rc = self._lib.co_init(self.device_id, ctypes.byref(self._handle))
        if rc != CO_OK:
            raise COError(rc, "co_init")

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.teardown()
        return False

    def _check(self):
        if self._torn:
            raise RuntimeError("InProcessCO used after teardown()")

    def _build_header(self, pop: dict) -> PopHeader:
        return _header(pop)

    def optimize(self, pop: dict, max_iter: int = 50) -> dict:
        """Reference-compatible fit: fp32 in, fp32 out (co_inproc.py:165-215)."""
        self._check()
        M, C = int(pop["M"]), int(pop["total_c"])
        h = _header(pop)
        nt, pnt = _arr(pop["nt"], np.int32)
        nv, pnv = _arr(pop["nv"], np.float32)
        ci, pci = _arr(pop["ci"], np.int32)
        me, pme = _metas(pop)
        nc, nx, ny = _counts(pop)
        c0, pc0 = _sized(pop["c_init"], np.float32, nc, "c_init")
        xs, pxs = _sized(pop["xs"], np.float32, nx, "xs")
        ym, pym = _sized(pop["ym"], np.float32, ny, "ym")
        c_final = np.zeros(max(C, 1), np.float32)
        status = np.zeros(max(M, 1), np.int32)
        loss_init = np.zeros(max(M, 1), np.float32)
        loss_final = np.zeros(max(M, 1), np.float32)
        rc = self._lib.co_optimize(self._handle, ctypes.byref(h), pnt, pnv, pci, pme, pc0, pxs,
                                   pym, int(max_iter), c_final.ctypes.data_as(_VP),
                                   status.ctypes.data_as(_VP), loss_init.ctypes.data_as(_VP),
                                   loss_final.ctypes.data_as(_VP))
        if rc != CO_OK:
            raise COError(rc, "co_optimize")
        return {"c_final": c_final[:C], "status": status[:M],
                "loss_init": loss_init[:M], "loss_final": loss_final[:M]}

    def optimize_ex(self, pop: dict, max_iter: int = 50, *, ad_mode: int = CO_AD_FORWARD,
                    precision: int = CO_PREC_FP64, lambda0: float = 1e-3, xtol: float = 1e-6,
                    fp64_guard: bool = True, partitions: int = 0, lm_order: int | None = None,
                    damping: int = CO_DAMP_RELATIVE,
                    tail_iter: int = 0, tail_partitions: int = 0, f32_range: bool = False,
                    c_init=None, xs=None, ym=None) -> dict:
        """fp64 fit; c_init/xs/ym override the pop's (fp32) arrays when given.
        partitions: point partitions per expression (0: by N). lm_order: None
        keeps the library's default (CO_ORDER_IMPROVE_FIRST for the ad
        library, CO_ORDER_CONVERGE_FIRST for fd). damping: the solve's variant
        (CO_DAMP_RELATIVE, CO_DAMP_TRUST_REGION with lambda0 typically
        CO_TRUST_REGION_LAMBDA0, CO_DAMP_PIVOT_FLOOR). f32_range: trial
        constants held in fp32 and losses in its range, as co_optimize fits."""
        self._check()
        M, C = int(pop["M"]), int(pop["total_c"])
        h = _header(pop)
        o = default_options(ad_mode=int(ad_mode), precision=int(precision),
                            max_iter=int(max_iter), lambda0=float(lambda0), xtol=float(xtol),
                            fp64_guard=1 if fp64_guard else 0, partitions=int(partitions),
                            tail_iter=int(tail_iter), tail_partitions=int(tail_partitions),
                            f32_range=1 if f32_range else 0)
        o.lm_order = self.default_order if lm_order is None else int(lm_order)
        o.damping = int(damping)
        nt, pnt = _arr(pop["nt"], np.int32)
        nv, pnv = _arr(pop["nv"], np.float32)
        ci, pci = _arr(pop["ci"], np.int32)
        me, pme = _metas(pop)
        nc, nx, ny = _counts(pop)
        c0, pc0 = _sized(pop["c_init"] if c_init is None else c_init, np.float64, nc, "c_init")
        x, px = _sized(pop["xs"] if xs is None else xs, np.float64, nx, "xs")
        y, py = _sized(pop["ym"] if ym is None else ym, np.float64, ny, "ym")
        out = {"c_final": np.zeros(max(C, 1)), "status": np.zeros(max(M, 1), np.int32),
               "loss_init": np.zeros(max(M, 1)), "loss_final": np.zeros(max(M, 1)),
               "iters": np.zeros(max(M, 1), np.int32)}
        rc = self._lib.co_optimize_ex(
            self._handle, ctypes.byref(o), ctypes.byref(h), pnt, pnv, pci, pme, pc0, px, py,
            *(out[k].ctypes.data_as(_VP) for k in
              ("c_final", "status", "loss_init", "loss_final", "iters")))
        if rc != CO_OK:
            raise COError(rc, "co_optimize_ex")
        out["c_final"] = out["c_final"][:C]
        for k in ("status", "loss_init", "loss_final", "iters"):
            out[k] = out[k][:M]
        return out

    def evaluate(self, pop: dict, c=None, xs=None, precision: int = CO_PREC_FP64) -> np.ndarray:
        """y[m, i] of every expression at constants c (default c_init)."""
        self._check()
        M, N = int(pop["M"]), int(pop["N"])
        h = _header(pop)
        nt, pnt = _arr(pop["nt"], np.int32)
        nv, pnv = _arr(pop["nv"], np.float32)
        ci, pci = _arr(pop["ci"], np.int32)
        me, pme = _metas(pop)
        cc, pcc = _arr(pop["c_init"] if c is None else c, np.float64)
        if cc.size == 0:
            cc, pcc = _arr(np.zeros(1), np.float64)
        x, px = _sized(pop["xs"] if xs is None else xs, np.float64, _counts(pop)[1], "xs")
        y = np.zeros((max(M, 1), max(N, 1)))
        rc = self._lib.co_eval_ex(self._handle, ctypes.byref(h), pnt, pnv, pci, pme, pcc, px,
                                  int(precision), y.ctypes.data_as(_VP))
        if rc != CO_OK:
            raise COError(rc, "co_eval_ex")
        return y[:M, :N]

    def upload(self, pop: dict, *, c_init=None, xs=None, ym=None) -> None:
        """Make pop resident on the device for fit_resident() (fp64 inputs)."""
        self._check()
        h = _header(pop)
        nt, pnt = _arr(pop["nt"], np.int32)
        nv, pnv = _arr(pop["nv"], np.float32)
        ci, pci = _arr(pop["ci"], np.int32)
        me, pme = _metas(pop)
        nc, nx, ny = _counts(pop)
        c0, pc0 = _sized(pop["c_init"] if c_init is None else c_init, np.float64, nc, "c_init")
        if c0.size == 0:
            c0, pc0 = _arr(np.zeros(1), np.float64)
        x, px = _sized(pop["xs"] if xs is None else xs, np.float64, nx, "xs")
        y, py = _sized(pop["ym"] if ym is None else ym, np.float64, ny, "ym")
        rc = self._lib.co_upload_ex(self._handle, ctypes.byref(h), pnt, pnv, pci, pme, pc0, px, py)
        if rc != CO_OK:
            raise COError(rc, "co_upload_ex")
        self._resident = (int(pop["M"]), int(pop["total_c"]))

    def upload_data(self, xs, y) -> None:
        """Keep one data set (xs [N, D], target y [N], fp64) on the device for
        optimize_data; it stays until the next upload_data or teardown."""
        self._check()
        x, px = _arr(xs, np.float64)
        yy, py = _arr(y, np.float64)
        if x.ndim != 2 or yy.size != x.shape[0]:
            raise ValueError(f"xs must be [N, D] and y [N]; got {x.shape} and {yy.shape}")
        self._data = None
        rc = self._lib.co_data_upload(self._handle, int(x.shape[0]), int(x.shape[1]), px, py)
        if rc != CO_OK:
            raise COError(rc, "co_data_upload")
        self._data = (x.copy(), yy.copy())

    def upload_data_device(self, xs, y) -> None:
        """upload_data from device tensors (torch, float64, contiguous, on this
        handle's device): xs [N, D] and y [N] are copied device to device,
        never through host memory. Waits for the current torch stream first,
        so the tensors are complete when the library reads them."""
        self._check()
        import torch

        if not (isinstance(xs, torch.Tensor) and isinstance(y, torch.Tensor)):
            raise TypeError("upload_data_device takes torch tensors")
        if xs.dtype != torch.float64 or y.dtype != torch.float64:
            raise ValueError("xs and y must be float64")
        if xs.dim() != 2 or y.dim() != 1 or y.shape[0] != xs.shape[0]:
            raise ValueError(f"xs must be [N, D] and y [N]; got {tuple(xs.shape)} and "
                             f"{tuple(y.shape)}")
        if not (xs.is_contiguous() and y.is_contiguous()):
            raise ValueError("xs and y must be contiguous")
        for t in (xs, y):
            if t.is_cuda:
                torch.cuda.current_stream(t.device).synchronize()
        self._data = None
        rc = self._lib.co_data_upload_device(self._handle, int(xs.shape[0]), int(xs.shape[1]),
                                             ctypes.c_void_p(xs.data_ptr()),
                                             ctypes.c_void_p(y.data_ptr()))
        if rc != CO_OK:
            raise COError(rc, "co_data_upload_device")

    def data_matches(self, xs, y) -> bool:
        """True when (xs, y) equal the uploaded data set value for value."""
        if self._data is None:
            return False
        x0, y0 = self._data
        xs, y = np.asarray(xs), np.asarray(y).ravel()
        return (xs.shape == x0.shape and y.shape == y0.shape and np.array_equal(xs, x0)
                and np.array_equal(y, y0))

    def optimize_data(self, pop: dict, max_iter: int = 50, *, ad_mode: int = CO_AD_FORWARD,
                      precision: int = CO_PREC_FP64, lambda0: float = 1e-3, xtol: float = 1e-6,
                      fp64_guard: bool = True, partitions: int = 0, lm_order: int | None = None,
                      damping: int = CO_DAMP_RELATIVE,
                    tail_iter: int = 0, tail_partitions: int = 0, f32_range: bool = False,
                      c_init=None) -> dict:
        """optimize_ex against the uploaded data set: pop's xs and ym are not
        read or sent; only the programs and constants go to the device."""
        self._check()
        M, C = int(pop["M"]), int(pop["total_c"])
        h = _header(pop)
        o = default_options(ad_mode=int(ad_mode), precision=int(precision),
                            max_iter=int(max_iter), lambda0=float(lambda0), xtol=float(xtol),
                            fp64_guard=1 if fp64_guard else 0, partitions=int(partitions),
                            tail_iter=int(tail_iter), tail_partitions=int(tail_partitions),
                            f32_range=1 if f32_range else 0)
        o.lm_order = self.default_order if lm_order is None else int(lm_order)
        o.damping = int(damping)
        nt, pnt = _arr(pop["nt"], np.int32)
        nv, pnv = _arr(pop["nv"], np.float32)
        ci, pci = _arr(pop["ci"], np.int32)
        me, pme = _metas(pop)
        c0, pc0 = _sized(pop["c_init"] if c_init is None else c_init, np.float64, C, "c_init")
        if c0.size == 0:
            c0, pc0 = _arr(np.zeros(1), np.float64)
        out = {"c_final": np.zeros(max(C, 1)), "status": np.zeros(max(M, 1), np.int32),
               "loss_init": np.zeros(max(M, 1)), "loss_final": np.zeros(max(M, 1)),
               "iters": np.zeros(max(M, 1), np.int32)}
        rc = self._lib.co_optimize_data(
            self._handle, ctypes.byref(o), ctypes.byref(h), pnt, pnv, pci, pme, pc0,
            *(out[k].ctypes.data_as(_VP) for k in
              ("c_final", "status", "loss_init", "loss_final", "iters")))
        if rc != CO_OK:
            raise COError(rc, "co_optimize_data")
        self._resident = (M, C)
        out["c_final"] = out["c_final"][:C]
        for k in ("status", "loss_init", "loss_final", "iters"):
            out[k] = out[k][:M]
        return out

    def optimize_data_device(self, pop: dict, c_init, max_iter: int = 50, *,
                             ad_mode: int = CO_AD_FORWARD, precision: int = CO_PREC_FP64,
                             lambda0: float = 1e-3, xtol: float = 1e-6, fp64_guard: bool = True,
                             partitions: int = 0, lm_order: int | None = None,
                             damping: int = CO_DAMP_RELATIVE,
                             f32_range: bool = False) -> dict:
        """optimize_data with the constants and results on the device
        (co_optimize_data_device): c_init is a float64 CUDA tensor of
        total_c values; returns CUDA tensors c_final (float64), status
        (int32), loss_init, loss_final (float64) and iters (int32) on its
        device. The programs go from pop (host) as in optimize_data."""
        import torch

        self._check()
        M, C = int(pop["M"]), int(pop["total_c"])
        if (not isinstance(c_init, torch.Tensor) or not c_init.is_cuda
                or c_init.dtype != torch.float64 or c_init.numel() != C):
            raise ValueError(f"c_init must be a float64 CUDA tensor of {C} values")
        dev = c_init.device
        c0 = c_init.contiguous()
        h = _header(pop)
        o = default_options(ad_mode=int(ad_mode), precision=int(precision),
                            max_iter=int(max_iter), lambda0=float(lambda0), xtol=float(xtol),
                            fp64_guard=1 if fp64_guard else 0, partitions=int(partitions),
                            f32_range=1 if f32_range else 0)
        o.lm_order = self.default_order if lm_order is None else int(lm_order)
        o.damping = int(damping)
        nt, pnt = _arr(pop["nt"], np.int32)
        nv, pnv = _arr(pop["nv"], np.float32)
        ci, pci = _arr(pop["ci"], np.int32)
        me, pme = _metas(pop)
        out = {"c_final": torch.empty(C, dtype=torch.float64, device=dev),
               "status": torch.empty(M, dtype=torch.int32, device=dev),
               "loss_init": torch.empty(M, dtype=torch.float64, device=dev),
               "loss_final": torch.empty(M, dtype=torch.float64, device=dev),
               "iters": torch.empty(M, dtype=torch.int32, device=dev)}
        # the library copies on its own stream: torch's work on these tensors
        # (the allocations, c_init's producer) is complete first
        torch.cuda.synchronize(dev)
        ptr = lambda t: ctypes.c_void_p(t.data_ptr() if t.numel() else 0)  # noqa: E731
        rc = self._lib.co_optimize_data_device(
            self._handle, ctypes.byref(o), ctypes.byref(h), pnt, pnv, pci, pme, ptr(c0),
            *(ptr(out[k]) for k in ("c_final", "status", "loss_init", "loss_final", "iters")))
        if rc != CO_OK:
            raise COError(rc, "co_optimize_data_device")
        self._resident = (M, C)
        return out

    def fit_resident(self, max_iter: int = 50, *, ad_mode: int = CO_AD_FORWARD,
                     precision: int = CO_PREC_FP64, lambda0: float = 1e-3, xtol: float = 1e-6,
                     fp64_guard: bool = True, outputs: bool = True, partitions: int = 0,
                     tail_iter: int = 0, tail_partitions: int = 0, f32_range: bool = False,
                     lm_order: int | None = None,
                     damping: int = CO_DAMP_RELATIVE, static_scratch: bool = False):
        """Fit the uploaded population again; outputs=False leaves results on the
        device. static_scratch: co_fit_resident_static, the same fit with its
        scratch in the library's fixed device array (no device allocation)."""
        self._check()
        M, C = self._resident
        fn = self._lib.co_fit_resident_static if static_scratch else self._lib.co_fit_resident
        name = "co_fit_resident_static" if static_scratch else "co_fit_resident"
        o = default_options(ad_mode=int(ad_mode), precision=int(precision),
                            max_iter=int(max_iter), lambda0=float(lambda0), xtol=float(xtol),
                            fp64_guard=1 if fp64_guard else 0, partitions=int(partitions),
                            tail_iter=int(tail_iter), tail_partitions=int(tail_partitions),
                            f32_range=1 if f32_range else 0)
        o.lm_order = self.default_order if lm_order is None else int(lm_order)
        o.damping = int(damping)
        if not outputs:
            rc = fn(self._handle, ctypes.byref(o), None, None, None, None, None)
            if rc != CO_OK:
                raise COError(rc, name)
            return None
        out = {"c_final": np.zeros(max(C, 1)), "status": np.zeros(max(M, 1), np.int32),
               "loss_init": np.zeros(max(M, 1)), "loss_final": np.zeros(max(M, 1)),
               "iters": np.zeros(max(M, 1), np.int32)}
        rc = fn(self._handle, ctypes.byref(o),
                *(out[k].ctypes.data_as(_VP) for k in
                  ("c_final", "status", "loss_init", "loss_final", "iters")))
        if rc != CO_OK:
            raise COError(rc, name)
        out["c_final"] = out["c_final"][:C]
        for k in ("status", "loss_init", "loss_final", "iters"):
            out[k] = out[k][:M]
        return out

    def last_kernel_ms(self) -> float:
        """Device time of the last fit (HIP events on the library's stream)."""
        v = ctypes.c_double(-1.0)
        rc = self._lib.co_last_kernel_ms(self._handle, ctypes.byref(v))
        if rc != CO_OK:
            raise COError(rc, "co_last_kernel_ms")
        return v.value

    def last_bin_ms(self) -> np.ndarray:
        """Per-bin kernel durations of the last fit (ms, -1 for empty bins):
        [k] the fast kernel of K = k, [CO_GENERAL_BIN] the general kernel."""
        v = (ctypes.c_double * CO_BINS)()
        rc = self._lib.co_last_bin_ms(self._handle, v)
        if rc != CO_OK:
            raise COError(rc, "co_last_bin_ms")
        return np.asarray(v[:], dtype=np.float64)

    def last_split(self):
        """(setup_ms, loop_ms) of the last fit on this process."""
        s, l = ctypes.c_double(-1.0), ctypes.c_double(-1.0)
        rc = self._lib.co_last_split(ctypes.byref(s), ctypes.byref(l))
        if rc != 0 or s.value < 0:
            return (None, None)
        return (s.value, l.value)

    def teardown(self):
        if self._torn:
            return
        if self._handle:
            self._lib.co_teardown(self._handle)
            self._handle = _VP()
        self._torn = True

    def __del__(self):
        try:
            self.teardown()
        except Exception:  # noqa: BLE001
            pass


_SINGLETONS: dict[tuple[int, str], InProcessCO] = {}
_LOCK = threading.Lock()
_ATEXIT = False


def _teardown_all() -> None:
    for co in list(_SINGLETONS.values()):
        try:
            co.teardown()
        except Exception:  # noqa: BLE001
            pass
    _SINGLETONS.clear()


def get_inproc_co(device_id: int = 0, variant: str = "fd") -> InProcessCO:
    """Process-wide InProcessCO per (device, variant) (co_inproc.py:271-295)."""
    global _ATEXIT
    key = (int(device_id), str(variant))
    with _LOCK:
        co = _SINGLETONS.get(key)
        if co is None or co._torn:
            co = InProcessCO(device_id=device_id, variant=variant)
            _SINGLETONS[key] = co
            if not _ATEXIT:
                atexit.register(_teardown_all)
                _ATEXIT = True
        return co
