"""pop.bin reader / writer / builder.

v1 has the byte layout and dict keys of the reference
(cusr/benchmark/popio.py:26-120, cusr/kernel/pop_format.h:6-51): a 64-byte
header of 16 int32 (magic, version, M, total_nodes, total_c, N, n_vars, K_max,
max_stack, 7 reserved), then nt i32[T], nv f32[T], ci i32[T], metas i32[M,4],
c_init f32[C], xs f32[N, n_vars] and ym f32[M, N].

v2 (extension, include/pop_format.h) sets version 2 and flags in reserved[0]:
POP_FLAG_F64 stores c_init, xs and ym as float64; POP_FLAG_SHARED_Y stores one
ym row that every expression fits (the dict then has shared_y=True and ym of
shape (1, N)). v1 files read and write as before.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

POP_MAGIC = 0x4D4C344D
POP_VERSION = 1
POP_VERSION_2 = 2
POP_FLAG_F64, POP_FLAG_SHARED_Y = 1, 2
HEADER_BYTES = 64

NODE_VAR, NODE_CONST, NODE_UFUNC, NODE_BFUNC = 0, 1, 2, 3

_KEYS = ("M", "total_nodes", "total_c", "N", "n_vars", "K_max", "max_stack")


def pop_bytes(M: int, T: int, C: int, N: int, D: int, flags: int = 0) -> int:
    """File size of a population (v1 when flags is 0)."""
    s = 8 if flags & POP_FLAG_F64 else 4
    rows = 1 if flags & POP_FLAG_SHARED_Y else M
    return HEADER_BYTES + 12 * T + 16 * M + s * C + s * N * D + s * rows * N


def load_pop_bin(path) -> dict:
    """Read a v1 or v2 file into the reference dict layout (popio.py:26-41)."""
    raw = Path(path).read_bytes()
    if len(raw) < HEADER_BYTES:
        raise ValueError(f"{path}: {len(raw)} bytes, shorter than the header")
    h = np.frombuffer(raw, dtype="<i4", count=16)
    magic, version, M, T, C, N, D, K_max, max_stack = (int(v) for v in h[:9])
    if magic != POP_MAGIC:
        raise ValueError(f"bad magic 0x{magic & 0xFFFFFFFF:08x} (want 0x{POP_MAGIC:08x})")
    if version not in (POP_VERSION, POP_VERSION_2):
        raise ValueError(f"version {version} is neither {POP_VERSION} nor {POP_VERSION_2}")
    flags = int(h[9]) if version == POP_VERSION_2 else 0
    if flags & ~(POP_FLAG_F64 | POP_FLAG_SHARED_Y):
        raise ValueError(f"unknown flags 0x{flags:x}")
    want = pop_bytes(M, T, C, N, D, flags)
    if len(raw) < want:
        raise ValueError(f"{path}: {len(raw)} bytes, header implies {want}")
    off = HEADER_BYTES

    def take(dtype, count, shape=None):
        nonlocal off
        a = np.frombuffer(raw, dtype=dtype, count=count, offset=off).copy()
        off += np.dtype(dtype).itemsize * count
        return a if shape is None else a.reshape(shape)

    fdt = "<f8" if flags & POP_FLAG_F64 else "<f4"
    rows = 1 if flags & POP_FLAG_SHARED_Y else M
    nt = take("<i4", T)
    nv = take("<f4", T)
    ci = take("<i4", T)
    metas = take("<i4", 4 * M, (M, 4))
    c_init = take(fdt, C)
    xs = take(fdt, N * D, (N, D))
    ym = take(fdt, rows * N, (rows, N))
    pop = dict(M=M, total_nodes=T, total_c=C, N=N, n_vars=D, K_max=K_max,
               max_stack=max_stack, nt=nt, nv=nv, ci=ci, metas=metas,
               c_init=c_init, xs=xs, ym=ym)
    if flags & POP_FLAG_SHARED_Y:
        pop["shared_y"] = True
    return pop


def header_array(pop: dict, flags: int = 0) -> np.ndarray:
    h = np.zeros(16, dtype="<i4")
    h[0], h[1] = POP_MAGIC, POP_VERSION_2 if flags else POP_VERSION
    h[2:9] = [int(pop[k]) for k in _KEYS]
    h[9] = flags
    return h


def save_pop_bin(pop: dict, path, f64: bool = False) -> None:
    """Write the dict layout: v1 (the reference's, popio.py:44-56) unless the
    population has a shared target or f64 is set, which write v2."""
    flags = (POP_FLAG_F64 if f64 else 0) | (POP_FLAG_SHARED_Y if pop.get("shared_y") else 0)
    fdt = "<f8" if f64 else "<f4"
    parts = [header_array(pop, flags).tobytes()]
    for key, dt in (("nt", "<i4"), ("nv", "<f4"), ("ci", "<i4"), ("metas", "<i4"),
                    ("c_init", fdt), ("xs", fdt), ("ym", fdt)):
        parts.append(np.ascontiguousarray(pop[key], dtype=dt).tobytes())
    Path(path).write_bytes(b"".join(parts))


def share_y(pop: dict) -> dict:
    """The same population with one shared target row (every row of ym must
    be equal)."""
    ym = np.asarray(pop["ym"])
    if not np.all(ym == ym[:1]):
        raise ValueError("rows of ym differ: the target is not shared")
    out = dict(pop)
    out["ym"] = ym[:1].copy()
    out["shared_y"] = True
    return out


def y_rows(pop: dict) -> np.ndarray:
    """ym with one row per expression (a shared row repeated)."""
    ym = np.asarray(pop["ym"])
    return np.broadcast_to(ym[:1], (int(pop["M"]), ym.shape[1])) if pop.get("shared_y") else ym


def stack_depth(nt) -> int:
    """Value-stack depth of one expression evaluated last node first."""
    nt = np.asarray(nt)
    step = np.where(nt <= NODE_CONST, 1, np.where(nt == NODE_BFUNC, -1, 0))
    return int(np.max(np.cumsum(step[::-1]))) if len(nt) else 0


def build_pop(trees, xs, ym) -> dict:
    """trees: [(nt, nv, ci, c_init)] -> pop dict with offsets, K_max, max_stack.

    Constant ranks must be 0..K-1 in prefix order (popio.py:87-91)."""
    xs = np.atleast_2d(np.asarray(xs, np.float32))
    nts, nvs, cis, cs, metas = [], [], [], [], []
    node_off = c_off = K_max = max_stack = 0
    for nt, nv, ci, c0 in trees:
        nt = np.asarray(nt, np.int32)
        ci = np.asarray(ci, np.int32)
        K = int(np.count_nonzero(nt == NODE_CONST))
        ranks = ci[nt == NODE_CONST]
        if not np.array_equal(ranks, np.arange(K)):
            raise ValueError(f"const ranks must be 0..{K - 1} in prefix order, got {ranks.tolist()}")
        c0 = np.asarray(c0, np.float32).ravel()
        if c0.size != K:
            raise ValueError(f"c_init has {c0.size} values, expression has K={K}")
        metas.append((node_off, len(nt), c_off, K))
        nts.append(nt)
        nvs.append(np.asarray(nv, np.float32))
        cis.append(ci)
        cs.append(c0)
        node_off += len(nt)
        c_off += K
        K_max = max(K_max, K)
        max_stack = max(max_stack, stack_depth(nt))
    M = len(metas)
    ym = np.asarray(ym, np.float32).reshape(M, xs.shape[0])
    return dict(M=M, total_nodes=node_off, total_c=c_off, N=xs.shape[0], n_vars=xs.shape[1],
                K_max=K_max, max_stack=max_stack,
                nt=np.concatenate(nts) if nts else np.zeros(0, np.int32),
                nv=np.concatenate(nvs) if nvs else np.zeros(0, np.float32),
                ci=np.concatenate(cis) if cis else np.zeros(0, np.int32),
                metas=np.asarray(metas, np.int32).reshape(-1, 4),
                c_init=np.concatenate(cs) if c_off else np.zeros(0, np.float32),
                xs=xs, ym=ym)


def tree_slices(pop: dict, m: int):
    """(nt, nv, ci, c_init, ym row, K) of expression m."""
    off, n, c_off, K = (int(v) for v in pop["metas"][m])
    sl = slice(off, off + n)
    return (pop["nt"][sl], pop["nv"][sl], pop["ci"][sl],
            pop["c_init"][c_off:c_off + K], y_rows(pop)[m], K)


def slice_pop(pop: dict, limit: int) -> dict:
    """The first `limit` expressions, offsets rebuilt (popio.py:109-120)."""
    if limit >= pop["M"]:
        return pop
    return select_pop(pop, np.arange(limit))


def select_pop(pop: dict, idx) -> dict:
    """Expressions idx (any order), offsets rebuilt."""
    idx = np.asarray(idx, dtype=np.int64)
    trees = [tree_slices(pop, int(m))[:4] for m in idx]
    out = build_pop(trees, pop["xs"], y_rows(pop)[idx])
    if np.asarray(pop["c_init"]).dtype == np.float64:
        # a float64 (v2) population keeps its exact payload
        out["c_init"] = np.concatenate([tree_slices(pop, int(m))[3] for m in idx]) \
            if out["total_c"] else np.zeros(0)
        out["xs"] = np.asarray(pop["xs"], np.float64)
        out["ym"] = np.asarray(y_rows(pop)[idx], np.float64)
    return share_y(out) if pop.get("shared_y") else out
