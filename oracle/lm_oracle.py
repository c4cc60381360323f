"""ctypes binding of the C oracle (lm_oracle.c). Test infrastructure only.

Functions take a pop dict (keys of the reference popio dict, popio.py:39-41)
and numpy arrays, and return numpy arrays. Data and constants are fp64.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
# CUSR_ORACLE_LIB names another build of the oracle (the mutation gate,
# oracle/mutation_gate.py, points the tests at mutant builds)
_LIB_PATH = Path(os.environ.get("CUSR_ORACLE_LIB") or (_HERE / "liblm_oracle.so"))
_lib = None

CO_AD_FORWARD, CO_AD_REVERSE = 0, 1
CO_PREC_FP64, CO_PREC_MIXED = 0, 1
# damped-solve variants (include/cusr_co.h CoOptions.damping)
CO_DAMP_RELATIVE, CO_DAMP_TRUST_REGION, CO_DAMP_PIVOT_FLOOR = 0, 1, 2
CO_PIVOT_FLOOR_EPS = float(np.float32(1e-9))
CO_TRUST_REGION_LAMBDA0 = float(np.float32(1e-4))


class PopHeader(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("magic", "version", "M_prob", "total_nodes", "total_c", "N",
                 "n_vars", "K_max", "max_stack")] + [("reserved", ctypes.c_int32 * 7)]


class CoOptions(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_int32), ("ad_mode", ctypes.c_int32),
                ("precision", ctypes.c_int32), ("max_iter", ctypes.c_int32),
                ("lambda0", ctypes.c_double), ("xtol", ctypes.c_double),
                ("fp64_guard", ctypes.c_int32), ("partitions", ctypes.c_int32),
                ("lm_order", ctypes.c_int32), ("tail_iter", ctypes.c_int32),
                ("tail_partitions", ctypes.c_int32), ("f32_range", ctypes.c_int32),
                ("damping", ctypes.c_int32), ("reserved", ctypes.c_int32)]


def build() -> None:
    """Compile liblm_oracle.so (and oracle/_ref when the reference is mounted)."""
    subprocess.run(["make", "-s", "-C", str(_HERE), "all"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
    return _lib


def _header(pop) -> PopHeader:
    h = PopHeader()
    h.magic, h.version = 0x4D4C344D, 1
    h.M_prob, h.total_nodes, h.total_c = int(pop["M"]), int(pop["total_nodes"]), int(pop["total_c"])
    h.N, h.n_vars, h.K_max, h.max_stack = (int(pop["N"]), int(pop["n_vars"]),
                                          int(pop["K_max"]), int(pop["max_stack"]))
    if pop.get("shared_y"):
        h.version, h.reserved[0] = 2, 2     # pop.bin v2, POP_FLAG_SHARED_Y
    return h


def _p(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a, a.ctypes.data_as(ctypes.c_void_p)


def _prog(pop):
    nt, pnt = _p(pop["nt"], np.int32)
    nv, pnv = _p(pop["nv"], np.float32)
    ci, pci = _p(pop["ci"], np.int32)
    me, pme = _p(pop["metas"], np.int32)
    return (nt, nv, ci, me), (pnt, pnv, pci, pme)


def options(ad_mode=CO_AD_FORWARD, precision=CO_PREC_FP64, max_iter=50,
            lambda0=1e-3, xtol=1e-6, fp64_guard=1, partitions=0, lm_order=0,
            tail_iter=0, tail_partitions=0, f32_range=0, damping=0) -> CoOptions:
    o = CoOptions()
    o.struct_size = ctypes.sizeof(CoOptions)
    o.ad_mode, o.precision, o.max_iter = ad_mode, precision, max_iter
    o.lambda0, o.xtol, o.fp64_guard = lambda0, xtol, fp64_guard
    o.partitions = partitions
    o.lm_order = lm_order
    o.tail_iter, o.tail_partitions = tail_iter, tail_partitions
    o.f32_range = f32_range
    o.damping = damping
    return o


def check_pop(pop):
    """(rc, stack depth per expression)."""
    keep, ptrs = _prog(pop)
    st = np.zeros(max(int(pop["M"]), 1), np.int32)
    h = _header(pop)
    rc = lib().orc_check_pop(ctypes.byref(h), *ptrs, st.ctypes.data_as(ctypes.c_void_p))
    return rc, st[: int(pop["M"])]


def fit(pop, *, c_init=None, xs=None, ym=None, **opt):
    """LM fit of every expression; returns dict like co_optimize_ex outputs."""
    o = options(**opt)
    keep, ptrs = _prog(pop)
    c0, pc0 = _p(pop["c_init"] if c_init is None else c_init, np.float64)
    x, px = _p(pop["xs"] if xs is None else xs, np.float64)
    y, py = _p(pop["ym"] if ym is None else ym, np.float64)
    M, C = int(pop["M"]), int(pop["total_c"])
    out = dict(c_final=np.zeros(max(C, 1)), status=np.zeros(max(M, 1), np.int32),
               loss_init=np.zeros(max(M, 1)), loss_final=np.zeros(max(M, 1)),
               iters=np.zeros(max(M, 1), np.int32))
    h = _header(pop)
    rc = lib().orc_fit(ctypes.byref(o), ctypes.byref(h), *ptrs, pc0, px, py,
                       *(out[k].ctypes.data_as(ctypes.c_void_p) for k in
                         ("c_final", "status", "loss_init", "loss_final", "iters")))
    if rc != 0:
        raise RuntimeError(f"orc_fit returned {rc}")
    out["c_final"] = out["c_final"][:C]
    for k in ("status", "loss_init", "loss_final", "iters"):
        out[k] = out[k][:M]
    return out


def eval_pop(pop, c=None, xs=None, precision=CO_PREC_FP64):
    keep, ptrs = _prog(pop)
    cc, pcc = _p(pop["c_init"] if c is None else c, np.float64)
    x, px = _p(pop["xs"] if xs is None else xs, np.float64)
    M, N = int(pop["M"]), int(pop["N"])
    y = np.zeros((M, N))
    h = _header(pop)
    rc = lib().orc_eval(ctypes.byref(h), *ptrs, pcc, px, ctypes.c_int(precision),
                        y.ctypes.data_as(ctypes.c_void_p))
    if rc != 0:
        raise RuntimeError(f"orc_eval returned {rc}")
    return y


def jacobian(pop, c=None, xs=None, ad_mode=CO_AD_FORWARD):
    """J[m, i, j] = d f_m(x_i) / d c_j (zero-padded to K_max)."""
    keep, ptrs = _prog(pop)
    cc, pcc = _p(pop["c_init"] if c is None else c, np.float64)
    x, px = _p(pop["xs"] if xs is None else xs, np.float64)
    M, N, KM = int(pop["M"]), int(pop["N"]), int(pop["K_max"])
    J = np.zeros((M, N, max(KM, 1)))
    h = _header(pop)
    rc = lib().orc_jacobian(ctypes.byref(h), *ptrs, pcc, px, ctypes.c_int(ad_mode),
                            J.ctypes.data_as(ctypes.c_void_p))
    if rc != 0:
        raise RuntimeError(f"orc_jacobian returned {rc}")
    return J[:, :, :KM]


def solve(jtj, jtr, lam, damping=0):
    """Damped Cholesky step of the oracle under damping variant `damping`
    (CoOptions.damping); None when the pivot rule fails the step."""
    K = len(jtr)
    a, pa = _p(np.triu(jtj), np.float64)
    b, pb = _p(jtr, np.float64)
    d = np.zeros(K)
    rc = lib().orc_solve_api(ctypes.c_int(K), pa, pb, ctypes.c_double(lam),
                             ctypes.c_int(damping), d.ctypes.data_as(ctypes.c_void_p))
    return None if rc != 0 else d


def pass_sums(pop, m, c, xs=None, y=None, precision=CO_PREC_FP64, ad_mode=CO_AD_FORWARD,
              partitions=0):
    """(loss, JtJ, Jtr) of expression m at constants c (canonical order)."""
    keep, ptrs = _prog(pop)
    K = int(pop["metas"][m][3])
    cc, pcc = _p(c, np.float64)
    x, px = _p(pop["xs"] if xs is None else xs, np.float64)
    yrow = pop["ym"][0] if pop.get("shared_y") else pop["ym"][m]
    yy, pyy = _p(yrow if y is None else y, np.float64)
    loss = ctypes.c_double()
    jtj = np.zeros((max(K, 1), max(K, 1)))
    jtr = np.zeros(max(K, 1))
    h = _header(pop)
    rc = lib().orc_pass_api(ctypes.byref(h), *ptrs, ctypes.c_int(m), pcc, px, pyy,
                            ctypes.c_int(precision), ctypes.c_int(ad_mode),
                            ctypes.c_int(partitions), ctypes.byref(loss),
                            jtj.ctypes.data_as(ctypes.c_void_p), jtr.ctypes.data_as(ctypes.c_void_p))
    if rc != 0:
        raise RuntimeError(f"orc_pass_api returned {rc}")
    return loss.value, jtj[:K, :K], jtr[:K]


MATH = {"exp": 0, "log": 1, "sin": 2, "cos": 3, "tan": 4, "sinh": 5, "cosh": 6, "tanh": 7,
        "pow": 8}


def math_fn(name, x, y=None, fp32=False):
    """include/cusr_math.h function `name` over arrays (fp32 variant if fp32)."""
    code = MATH[name] + (16 if fp32 else 0)
    xa, px = _p(x, np.float64)
    ya, py = (_p(y, np.float64) if y is not None else (None, None))
    out = np.zeros(xa.size)
    rc = lib().orc_math(ctypes.c_int(code), ctypes.c_int(xa.size), px, py,
                        out.ctypes.data_as(ctypes.c_void_p))
    if rc != 0:
        raise RuntimeError(f"orc_math returned {rc}")
    return out
