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
  * shapes that do not match raise ValueError.
Prints "torch interop ok" on success, exits non-zero otherwise.
"""
import ctypes
import sys
from pathlib import Path

import numpy as np
import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

from cusr_amd.kernel import co_inproc as ci  # noqa: E402
from tests.helpers import synth  # noqa: E402


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
    finally:
        co.teardown()
    print("torch interop ok", flush=True)


if __name__ == "__main__":
    main()
