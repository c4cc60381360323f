"""Writes tests/golden/scipy_pop1000.npz: the scipy CPU path on the reference's
real EvoGP population (tests/golden/ref_fixtures/pop1000.bin, N = 1,000,
D = 3), for the release gate of tests/test_gpu_reference_data.py.

Runs this repository's restatement of the reference ScipyPop backend
(oracle/scipy_pop.py; cusr/benchmark/backends.py:97-162): one
least_squares(method='lm', xtol=1e-10, ftol=1e-10, max_nfev=200) per K > 0
expression from the file's float32 c_init promoted to float64. The losses are
rescored with the numpy fp64 interpreter (oracle/interp.py), as the
reference's verify.py rescores every backend (cusr/kernel/verify.py:181-215).
The scipy fit of 1,000 expressions takes minutes of CPU, so it runs here once
and the result is committed; the GPU test only reads it.

    python tests/golden/make_scipy_pop1000.py [--nproc N]
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from cusr_amd.benchmark import popio  # noqa: E402
from oracle import interp, scipy_pop  # noqa: E402

OUT = HERE / "scipy_pop1000.npz"


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--nproc", type=int, default=None)
    a = ap.parse_args()
    pop = popio.load_pop_bin(HERE / "ref_fixtures" / "pop1000.bin")
    sp = scipy_pop.ScipyPop(nproc=a.nproc, timeout=600.0)
    try:
        r = sp.fit_pop(pop)
    finally:
        sp.close()
    loss = interp.loss_pop(pop, r["c_final"])
    np.savez_compressed(OUT, c_final=r["c_final"], status=r["status"], nfev=r["n_iter"],
                        loss=loss)
    print(f"{OUT.name}: {r['n_fit']} fits in {r['wall_core']:.1f} s on {r['nproc']} processes; "
          f"status counts {np.bincount(r['status'], minlength=4).tolist()}")


if __name__ == "__main__":
    main()
