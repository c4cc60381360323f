"""The drop-in boundary on the GPU: the reference fp32 ABI (co_optimize), the
CLI and its blobs, handle reuse across shrinking/growing populations, edge
populations, and the FD variant's LM ordering -- each against the CPU oracle.

Reference behaviour followed: cusr/kernel/co_lib.h:45-71 (ABI, ownership),
cusr/kernel/tests/test_inproc_reuse.py:313,425-469 (reuse, status branches),
cusr/kernel/batch_lm_ad.cu:226-536 (CLI arguments, blobs, completion line).
"""
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from cusr_amd.benchmark import popio
from cusr_amd.kernel import co_inproc as ci
from oracle import lm_oracle
from tests.helpers import assert_parity, rel_diff, synth

pytestmark = pytest.mark.gpu
KDIR = Path(ci.__file__).resolve().parent


def _say(msg):
    print(msg, flush=True)


def test_reference_abi_fp32_outputs(co):
    """co_optimize: fp32 in/out; the fit runs in fp64 and its results go through
    the fp32 carrier (co_narrow_fp32): no constant overflowed to +-inf comes
    back, and an expression that would get one keeps its c_init."""
    pop, _ = synth("C1", 128, 256)
    _say("co_optimize fp32 C1 M=128 N=256")
    g = co.optimize(pop, 20)
    fit = lm_oracle.fit(pop, max_iter=20, f32_range=1)
    o = ci.narrow_fp32(pop, fit)
    assert g["c_final"].dtype == np.float32 and g["loss_final"].dtype == np.float32
    same = np.mean(g["c_final"] == o["c_final"])
    _say(f"fp32 constants equal to the narrowed oracle: {same:.4f}; demoted {o['demoted']}")
    # constants held in fp32 by the fit: the carrier is exact, nothing overflows
    assert o["demoted"] == 0 and np.array_equal(o["c_final"], fit["c_final"])
    assert np.all(np.isfinite(g["c_final"]))
    assert np.array_equal(g["c_final"], o["c_final"])
    assert np.array_equal(g["status"], o["status"])
    assert np.allclose(g["loss_final"], o["loss_final"], rtol=1e-6)


def test_handle_reuse_shrink_and_grow(co):
    """Buffers grow by capacity and never shrink; every call starts from its
    own c_init (test_inproc_reuse.py:313)."""
    big, _ = synth("C2", 256, 512)
    small, _ = synth("C1", 32, 128)
    highk, _ = synth("C3", 16, 256)
    runs = []
    for pop, kw in ((big, {}), (small, {}), (highk, {"ad_mode": 1}), (big, {}), (small, {})):
        _say(f"reuse M={pop['M']} N={pop['N']} {kw}")
        runs.append(co.optimize_ex(pop, 10, **kw))
    for a, b in ((runs[0], runs[3]), (runs[1], runs[4])):
        assert np.array_equal(a["c_final"], b["c_final"])
        assert np.array_equal(a["status"], b["status"])
    o = lm_oracle.fit(highk, max_iter=10, ad_mode=1)
    assert_parity(runs[2], o, 1e-9, "reuse high K reverse", exact=True)


def test_edge_populations(co):
    """All-K0 population (K0_SKIP, no iterations) and one-point data."""
    trees = [([3, 0, 0], [1.0, 0.0, 1.0], [-1, -1, -1], np.zeros(0, np.float32))] * 5
    xs = np.linspace(-1, 1, 70).reshape(35, 2)
    pop = popio.build_pop(trees, xs, np.ones((5, 35)))
    _say("K=0 population")
    r = co.optimize_ex(pop, 10)
    assert np.all(r["status"] == ci.STATUS_K0_SKIP) and np.all(r["iters"] == 0)
    o = lm_oracle.fit(pop, max_iter=10)
    assert np.array_equal(r["loss_init"], o["loss_init"])
    one, _ = synth("C1", 8, 1)
    _say("N=1 population")
    g = co.optimize_ex(one, 5)
    o = lm_oracle.fit(one, max_iter=5)
    assert np.array_equal(g["status"], o["status"])
    assert np.mean(rel_diff(g["loss_final"], o["loss_final"]) <= 1e-9) == 1.0


def test_errors_before_any_copy(co):
    pop, _ = synth("C1", 8, 16)
    bad = dict(pop)
    bad["total_c"] = int(pop["total_c"]) + 1
    # host arrays sized to the header, so the library's own check is reached
    bad["c_init"] = np.append(pop["c_init"], np.float32(0))
    with pytest.raises(ci.COError) as e:
        co.optimize_ex(bad, 5)
    assert e.value.code == ci.CO_ERR_SUM_C
    # the handle still works afterwards
    r = co.optimize_ex(pop, 5)
    assert r["status"].shape == (8,)


def test_fd_ordering_matches_oracle():
    """libcusr_co_fd.so: the FD variant's ordering by default (co_lib.cu:457-473)."""
    fd = ci.get_inproc_co(0, "fd")
    assert fd.default_order == ci.CO_ORDER_CONVERGE_FIRST
    pop, _ = synth("C2", 128, 512)
    _say("fd ordering C2 M=128 N=512")
    g = fd.optimize_ex(pop, 20, xtol=1e-4)
    o = lm_oracle.fit(pop, max_iter=20, xtol=1e-4, lm_order=1)
    assert_parity(g, o, 1e-9, "fd ordering", exact=True)


@pytest.mark.parametrize("exe,order", [("batch_lm_ad", 0), ("batch_lm", 1)])
def test_cli_blobs_and_completion_line(tmp_path, exe, order):
    """CLI arguments, output blobs and the completion line the benchmark
    parses (cusr/benchmark/backends.py:745,773-774)."""
    pop, _ = synth("C1", 64, 128)
    path = tmp_path / "pop.bin"
    popio.save_pop_bin(pop, path)
    _say(f"cli {exe}")
    r = subprocess.run([str(KDIR / exe), str(path), str(tmp_path), "--max-iter", "15"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert re.search(r"总耗时 ([\d.]+) 秒", r.stdout)
    status = np.fromfile(tmp_path / "status.bin", np.int32)
    c_final = np.fromfile(tmp_path / "c_final.bin", np.float32)
    lf = np.fromfile(tmp_path / "loss_final.bin", np.float32)
    li = np.fromfile(tmp_path / "loss_init.bin", np.float32)
    assert status.shape == (64,) and c_final.shape == (int(pop["total_c"]),)
    assert lf.shape == li.shape == (64,)
    o = ci.narrow_fp32(pop, lm_oracle.fit(pop, max_iter=15, lm_order=order, f32_range=1))
    _say(f"cli: statuses equal {np.mean(status == o['status']):.4f}; constants equal "
         f"{np.mean(c_final == o['c_final']):.4f}")
    assert np.array_equal(status, o["status"])
    assert np.array_equal(c_final, o["c_final"])
    assert np.array_equal(lf, o["loss_final"]) or np.allclose(lf, o["loss_final"], rtol=1e-6)
    # load failure exits 1
    bad = subprocess.run([str(KDIR / exe), str(tmp_path / "missing.bin")], capture_output=True,
                         timeout=60)
    assert bad.returncode == 1


@pytest.mark.parametrize("flag,damping", [("--trust-region", 1), ("--pivot-floor", 2)])
def test_cli_damping_flags(tmp_path, flag, damping):
    """--trust-region is the reference's batch_lm_ad_tr build (absolute damping
    from lambda 1e-4f, cusr/kernel/Makefile:57-63, batch_lm_ad.cu:152-172,
    301-306); --pivot-floor its -DPIVOT_FLOOR build: the blobs equal the
    oracle's fit under the same variant."""
    pop, _ = synth("C2", 64, 128)
    path = tmp_path / "pop.bin"
    popio.save_pop_bin(pop, path)
    _say(f"cli batch_lm_ad {flag}")
    r = subprocess.run([str(KDIR / "batch_lm_ad"), str(path), str(tmp_path), "--max-iter", "15",
                        flag], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    status = np.fromfile(tmp_path / "status.bin", np.int32)
    c_final = np.fromfile(tmp_path / "c_final.bin", np.float32)
    lam0 = lm_oracle.CO_TRUST_REGION_LAMBDA0 if damping == 1 else 1e-3
    o = ci.narrow_fp32(pop, lm_oracle.fit(pop, max_iter=15, f32_range=1, damping=damping,
                                          lambda0=lam0))
    _say(f"cli {flag}: statuses equal {np.mean(status == o['status']):.4f}; constants equal "
         f"{np.mean(c_final == o['c_final']):.4f}")
    assert np.array_equal(status, o["status"])
    assert np.array_equal(c_final, o["c_final"])


def _shared_target(M=96, N=256, seed=9):
    pop, _ = synth("C1", M, N)
    y = np.random.default_rng(seed).normal(size=N).astype(np.float32)
    tiled = dict(pop)
    tiled["ym"] = np.broadcast_to(y, (M, N)).copy()
    return tiled


@pytest.mark.parametrize("ad_mode", [0, 1])
def test_shared_target_equals_tiled(co, ad_mode):
    """pop.bin v2 shared target: one y row on the device gives the fit of the
    target repeated per expression, bit for bit, and the oracle's."""
    tiled = _shared_target()
    shared = popio.share_y(tiled)
    _say(f"shared target ad_mode={ad_mode}")
    a = co.optimize_ex(tiled, 30, ad_mode=ad_mode)
    b = co.optimize_ex(shared, 30, ad_mode=ad_mode)
    for k in ("c_final", "status", "loss_init", "loss_final", "iters"):
        assert np.array_equal(a[k], b[k], equal_nan=True), k
    o = lm_oracle.fit(shared, max_iter=30, ad_mode=ad_mode)
    assert_parity(b, o, 1e-9, f"shared target ad={ad_mode}", exact=True)
    # fp32 reference ABI (forward AD) and the resident path read the shared
    # row as well
    r = co.optimize(shared, 30)
    assert np.array_equal(r["status"], co.optimize_ex(tiled, 30, f32_range=True)["status"])
    co.upload(shared)
    res = co.fit_resident(30, ad_mode=ad_mode)
    assert np.array_equal(res["c_final"], a["c_final"], equal_nan=True)
    # a ym whose size disagrees with the flag is refused before any copy
    with pytest.raises(ValueError, match="ym has"):
        co.optimize_ex(dict(tiled, ym=shared["ym"]), 30)


def test_cli_reads_v2_f64_shared(tmp_path):
    """The CLI reads a v2 file with float64 payloads and a shared target and
    fits what the library fits from the same fp64 arrays."""
    shared = dict(popio.share_y(_shared_target(M=64, N=128)))
    for k in ("c_init", "xs", "ym"):
        shared[k] = np.asarray(shared[k], np.float64) * (1 + 2.0 ** -30)
    path = tmp_path / "pop.bin"
    popio.save_pop_bin(shared, path, f64=True)
    _say("cli batch_lm_ad v2")
    r = subprocess.run([str(KDIR / "batch_lm_ad"), str(path), str(tmp_path), "--max-iter", "20"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    status = np.fromfile(tmp_path / "status.bin", np.int32)
    c_final = np.fromfile(tmp_path / "c_final.bin", np.float32)
    # a float64 file fits in full fp64; its float32 blobs go through the carrier
    o = ci.narrow_fp32(shared, lm_oracle.fit(shared, max_iter=20))
    _say(f"cli v2: statuses equal {np.mean(status == o['status']):.4f}; constants equal "
         f"{np.mean(c_final == o['c_final']):.4f}")
    assert np.array_equal(status, o["status"])
    assert np.array_equal(c_final, o["c_final"])


@pytest.mark.parametrize("ad_mode,precision", [(0, 0), (1, 0), (0, 1)])
def test_resident_data_equals_tiled(co, ad_mode, precision):
    """co_data_upload + co_optimize_data: populations of different sizes fit
    against one uploaded (X, y) give the fits of optimize_ex with y tiled,
    bit for bit, also after other entry points used the handle in between."""
    base = _shared_target(M=80, N=300, seed=12)
    X, y = base["xs"].astype(np.float64), base["ym"][0].astype(np.float64)
    _say(f"resident data ad_mode={ad_mode} precision={precision}")
    co.upload_data(X, y)
    for M, seed in ((80, None), (33, 44)):
        pop = base if seed is None else dict(synth("C1", M, 300, seed=seed)[0])
        pop = dict(pop, xs=base["xs"], ym=np.tile(base["ym"][0], (M, 1)))
        want = co.optimize_ex(pop, 25, ad_mode=ad_mode, precision=precision)
        co.evaluate(synth("C2", 16, 64)[0])      # other work on the handle in between
        got = co.optimize_data(pop, 25, ad_mode=ad_mode, precision=precision)
        for k in ("c_final", "status", "loss_init", "loss_final", "iters"):
            assert np.array_equal(got[k], want[k], equal_nan=True), (M, k)
        # the population stays resident on the data set for co_fit_resident
        again = co.fit_resident(25, ad_mode=ad_mode, precision=precision)
        assert np.array_equal(again["c_final"], want["c_final"], equal_nan=True)


def test_resident_data_errors(co):
    pop, _ = synth("C1", 8, 40)
    fresh = ci.InProcessCO(device_id=0, variant="ad")
    try:
        with pytest.raises(ci.COError) as e:
            fresh.optimize_data(pop, 5)                 # nothing uploaded
        assert e.value.code == ci.CO_ERR_DATA
        fresh.upload_data(pop["xs"], pop["ym"][0])
        other, _ = synth("C1", 8, 41)
        with pytest.raises(ci.COError) as e:
            fresh.optimize_data(other, 5)               # N differs
        assert e.value.code == ci.CO_ERR_DATA
        r = fresh.optimize_data(pop, 5)
        assert r["status"].shape == (8,)
    finally:
        fresh.teardown()
    with pytest.raises(ValueError):
        co.upload_data(np.zeros((10, 2)), np.zeros(9))


def test_resident_data_from_device_tensors():
    """co_data_upload_device from torch CUDA tensors equals co_data_upload from
    host arrays bit for bit; host pointers are refused with CO_ERR_DATA. Runs
    in a child process (tests/torch_interop_check.py) that imports torch
    before loading the library, so both share torch's HIP runtime: this test
    process loaded the library first and holds the system runtime."""
    import subprocess
    import sys
    from pathlib import Path

    script = Path(__file__).resolve().parent / "torch_interop_check.py"
    _say("resident data from device tensors (child process, torch first)")
    r = subprocess.run([sys.executable, "-u", str(script)], capture_output=True, text=True,
                       timeout=180)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "torch interop ok" in r.stdout
