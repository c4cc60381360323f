"""Child-process check behind test_gpu_boundary.test_resident_data_from_device_tensors.

torch loads its own HIP runtime (libamdhip64 from torch/lib, soname
libamdhip64.so.7). The fitter library asks for that soname, so it shares
torch's runtime when torch is imported first; a process that loaded the
library first holds a second runtime and torch sees no GPU. This script runs
in a fresh process in torch-first order (the order of a torch-based caller),
uploads one data set from host arrays and from CUDA tensors, and checks:
  * the fits against both are equal bit for bit;
  * host memory passed as device pointers is refused with CO_ERR_DATA and the
    previous data set stays;
  * shapes that do not match raise ValueError;
  * the fit with constants in and results out in device memory
    (co_optimize_data_device) equals the host-buffer fit bit for bit, and
    host memory passed as the constants is refused with CO_ERR_DATA before
    anything is written;
  * the same equality on the library's other paths: a population of 16,384
    expressions (decoded and fitted in pipelined ranges, c_dev copied on the
    copy stream), 16 point partitions (the split path) and expressions of
    the general kernel (K > 16);
  * the C entry point called straight after a torch stream queued the write
    of c_dev behind other work (no synchronisation by the caller) reads the
    finished constants: the library waits for the process's queued work.
Prints "torch interop ok" on success, exits non-zero otherwise.
"""
import ctypes
import sys
from pathlib import Path

import numpy as np
import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

from cusr_amd.kernel import co_inproc as ci  # noqa: E402
from tests.general_pops import general_pop  # noqa: E402
from tests.helpers import synth  # noqa: E402

OUT_KEYS = ("c_final", "status", "loss_init", "loss_final", "iters")


def _device_route_equals_host(co, dev, pop, max_iter, label, **kw):
    """optimize_data_device against optimize_data on the uploaded data set."""
    print(f"case {label}: M={pop['M']} N={pop['N']} {kw}", flush=True)
    want = co.optimize_data(pop, max_iter, **kw)
    c_dev = torch.from_numpy(pop["c_init"].astype(np.float64)).to(dev)
    got = co.optimize_data_device(pop, c_dev, max_iter, **kw)
    for k in OUT_KEYS:
        assert np.array_equal(got[k].cpu().numpy(), want[k], equal_nan=True), (label, k)
    return want


def _raw_device_call(co, pop, max_iter, c_dev, outs):
    """co_optimize_data_device through ctypes, without the Python wrapper's
    synchronisation."""
    h = ci._header(pop)
    o = ci.default_options(max_iter=max_iter)
    o.lm_order = co.default_order
    keep = [ci._arr(pop["nt"], np.int32), ci._arr(pop["nv"], np.float32),
            ci._arr(pop["ci"], np.int32), ci._metas(pop)]
    vp = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    return co._lib.co_optimize_data_device(co._handle, ctypes.byref(o), ctypes.byref(h),
                                           *(k[1] for k in keep), vp(c_dev),
                                           *(vp(outs[k]) for k in OUT_KEYS))


def other_paths(co, dev):
    N = 600
    y = np.random.default_rng(5).normal(size=N).astype(np.float32).astype(np.float64)
    big, _ = synth("C1", 16384, N, seed=31)
    co.upload_data(big["xs"].astype(np.float64), y)
    _device_route_equals_host(co, dev, big, 12, "pipelined ranges")
    pop, _ = synth("C2", 64, N, seed=32)
    co.upload_data(pop["xs"].astype(np.float64), y)
    _device_route_equals_host(co, dev, pop, 12, "split path", partitions=16)
    gpop, _ = general_pop("highk", 24, N)
    co.upload_data(gpop["xs"].astype(np.float64), y)
    _device_route_equals_host(co, dev, gpop, 10, "general kernel")

    # ordering: the write of c_dev is queued on a torch stream behind a few
    # large products; the C call follows at once
    want = co.optimize_data(gpop, 10)
    C, M = int(gpop["total_c"]), int(gpop["M"])
    src = torch.from_numpy(gpop["c_init"].astype(np.float64)).to(dev)
    c_dev = torch.zeros(C, dtype=torch.float64, device=dev)
    outs = {k: torch.zeros(C if k == "c_final" else M,
                           dtype=torch.float64 if "loss" in k or k == "c_final" else torch.int32,
                           device=dev) for k in OUT_KEYS}
    a = torch.rand(4096, 4096, device=dev)
    torch.cuda.synchronize(dev)
    side = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(side):
        for _ in range(8):
            a = torch.mm(a, a) * 1e-3
        c_dev.copy_(src)
    rc = _raw_device_call(co, gpop, 10, c_dev, outs)
    assert rc == ci.CO_OK, rc
    torch.cuda.synchronize(dev)
    for k in OUT_KEYS:
        assert np.array_equal(outs[k].cpu().numpy(), want[k], equal_nan=True), ("ordering", k)
    print("case ordering: the queued c_dev write was complete when read", flush=True)


def main():
    dev = torch.device("cuda", 0)
    torch.zeros(1, device=dev)                 # torch's runtime owns the device first
    co = ci.InProcessCO(device_id=0, variant="ad")
    try:
        pop, _ = synth("C1", 48, 300)
        X = pop["xs"].astype(np.float64)
        y = np.random.default_rng(21).normal(size=300)
        pop = dict(pop, ym=np.tile(y.astype(np.float32), (48, 1)))
        y = y.astype(np.float32).astype(np.float64)
        co.upload_data(X, y)
        want = co.optimize_data(pop, 20)
        co.upload_data_device(torch.from_numpy(X).to(dev), torch.from_numpy(y).to(dev))
        got = co.optimize_data(pop, 20)
        for k in ("c_final", "status", "loss_init", "loss_final", "iters"):
            assert np.array_equal(got[k], want[k], equal_nan=True), k
        hx, hy = np.ascontiguousarray(X), np.ascontiguousarray(y)
        rc = co._lib.co_data_upload_device(co._handle, hx.shape[0], hx.shape[1],
                                            hx.ctypes.data_as(ctypes.c_void_p),
                                            hy.ctypes.data_as(ctypes.c_void_p))
        assert rc == ci.CO_ERR_DATA, rc
        again = co.optimize_data(pop, 20)
        assert np.array_equal(again["loss_final"], want["loss_final"], equal_nan=True)
        try:
            co.upload_data_device(torch.zeros((10, 2), dtype=torch.float64, device=dev),
                                  torch.zeros(9, dtype=torch.float64, device=dev))
            raise AssertionError("mismatched shapes accepted")
        except ValueError:
            pass
        # constants in and results out in device memory (co_optimize_data_device)
        c_dev = torch.from_numpy(pop["c_init"].astype(np.float64)).to(dev)
        dout = co.optimize_data_device(pop, c_dev, 20)
        for k in ("c_final", "status", "loss_init", "loss_final", "iters"):
            assert dout[k].is_cuda, k
            assert np.array_equal(dout[k].cpu().numpy(), want[k], equal_nan=True), k
        assert torch.equal(c_dev.cpu(), torch.from_numpy(pop["c_init"].astype(np.float64)))
        # host memory passed as the constants is refused before anything is
        # copied (the outputs stay as they were)
        h = ci._header(pop)
        o = ci.default_options(max_iter=20)
        o.lm_order = co.default_order
        keep = [ci._arr(pop["nt"], np.int32), ci._arr(pop["nv"], np.float32),
                ci._arr(pop["ci"], np.int32), ci._metas(pop)]
        C, M = int(pop["total_c"]), int(pop["M"])
        hc = np.ascontiguousarray(pop["c_init"].astype(np.float64))
        st = torch.full((M,), -5, dtype=torch.int32, device=dev)
        cf = torch.full((C,), 7.0, dtype=torch.float64, device=dev)
        vp = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        rc = co._lib.co_optimize_data_device(co._handle, ctypes.byref(o), ctypes.byref(h),
                                             *(k[1] for k in keep),
                                             hc.ctypes.data_as(ctypes.c_void_p), vp(cf), vp(st),
                                             None, None, None)
        assert rc == ci.CO_ERR_DATA, rc
        assert bool((cf.cpu() == 7.0).all()) and bool((st.cpu() == -5).all())
        other_paths(co, dev)
    finally:
        co.teardown()
    print("torch interop ok", flush=True)


if __name__ == "__main__":
    main()
