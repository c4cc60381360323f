"""pop.bin v1 and the v2 extension (include/pop_format.h): byte layout, round
trips, and the shared-target fit against the tiled one in the oracle.

v1 is the reference's layout (cusr/benchmark/popio.py:26-56,
cusr/kernel/pop_format.h:6-51); v2 adds float64 payloads and a shared target
row, flagged in reserved[0].
"""
import numpy as np
import pytest

from cusr_amd.benchmark import popio
from oracle import lm_oracle
from tests.helpers import REF_FIX, ref_pop, synth

V1_FIXTURES = ["pop_fixture.bin"]


def _same(a, b):
    for k in ("M", "total_nodes", "total_c", "N", "n_vars", "K_max", "max_stack"):
        assert int(a[k]) == int(b[k]), k
    for k in ("nt", "nv", "ci", "metas", "c_init", "xs", "ym"):
        x, y = np.asarray(a[k]), np.asarray(b[k])
        assert x.shape == y.shape and x.dtype == y.dtype, k
        assert np.array_equal(x.view(np.uint8), y.view(np.uint8)), k


def _shared_pop(M=48, N=96, seed=5):
    """A population whose rows of ym are one target (every expression fits y)."""
    pop, _ = synth("C1", M, N)
    rng = np.random.default_rng(seed)
    y = rng.normal(size=N).astype(np.float32)
    tiled = dict(pop)
    tiled["ym"] = np.broadcast_to(y, (M, N)).copy()
    return tiled


def test_v1_bytes_unchanged(tmp_path):
    """A v1 population writes the same bytes it was read from."""
    pop = ref_pop(V1_FIXTURES[0])
    out = tmp_path / "v1.bin"
    popio.save_pop_bin(pop, out)
    assert out.read_bytes() == (REF_FIX / V1_FIXTURES[0]).read_bytes()
    assert np.frombuffer(out.read_bytes()[:8], "<i4")[1] == popio.POP_VERSION


@pytest.mark.parametrize("f64", [False, True])
@pytest.mark.parametrize("shared", [False, True])
def test_v2_round_trip(tmp_path, f64, shared):
    tiled = _shared_pop()
    pop = popio.share_y(tiled) if shared else tiled
    if f64:
        pop = dict(pop)
        for k in ("c_init", "xs", "ym"):
            pop[k] = np.asarray(pop[k], np.float64) * (1 + 2.0 ** -40)   # not fp32-representable
    path = tmp_path / "pop.bin"
    popio.save_pop_bin(pop, path, f64=f64)
    raw = path.read_bytes()
    flags = (popio.POP_FLAG_F64 if f64 else 0) | (popio.POP_FLAG_SHARED_Y if shared else 0)
    M, T, C, N, D = (int(pop[k]) for k in ("M", "total_nodes", "total_c", "N", "n_vars"))
    assert len(raw) == popio.pop_bytes(M, T, C, N, D, flags)
    h = np.frombuffer(raw[:64], "<i4")
    assert h[1] == (popio.POP_VERSION_2 if flags else popio.POP_VERSION) and h[9] == flags
    back = popio.load_pop_bin(path)
    _same(back, pop if f64 else {**pop, **{k: np.asarray(pop[k], np.float32)
                                           for k in ("c_init", "xs", "ym")}})
    assert bool(back.get("shared_y")) == shared
    want = np.broadcast_to(np.asarray(pop["ym"], back["ym"].dtype)[:1], (M, N))
    assert np.array_equal(popio.y_rows(back), want)


def test_v2_rejects_unknown_flags_and_short_files(tmp_path):
    pop = popio.share_y(_shared_pop())
    path = tmp_path / "pop.bin"
    popio.save_pop_bin(pop, path)
    raw = bytearray(path.read_bytes())
    (tmp_path / "short.bin").write_bytes(bytes(raw[:-4]))
    with pytest.raises(ValueError, match="header implies"):
        popio.load_pop_bin(tmp_path / "short.bin")
    raw[36:40] = np.int32(4).tobytes()
    (tmp_path / "flags.bin").write_bytes(bytes(raw))
    with pytest.raises(ValueError, match="unknown flags"):
        popio.load_pop_bin(tmp_path / "flags.bin")
    with pytest.raises(ValueError, match="not shared"):
        popio.share_y(synth("C1", 8, 32)[0])


def test_select_keeps_f64_and_shared():
    tiled = _shared_pop()
    pop = dict(popio.share_y(tiled))
    for k in ("c_init", "xs", "ym"):
        pop[k] = np.asarray(pop[k], np.float64) * (1 + 2.0 ** -40)
    sub = popio.select_pop(pop, [5, 2, 9])
    assert sub["shared_y"] and sub["ym"].shape == (1, pop["N"])
    assert sub["c_init"].dtype == np.float64
    for j, m in enumerate((5, 2, 9)):
        a, b = popio.tree_slices(sub, j), popio.tree_slices(pop, m)
        for x, y in zip(a[:5], b[:5]):
            assert np.array_equal(x, y)


@pytest.mark.parametrize("ad_mode", [0, 1])
def test_oracle_shared_target_equals_tiled(ad_mode):
    """The oracle's fit of a shared-target population is bit-identical to the
    same fit with the target repeated per expression."""
    tiled = _shared_pop()
    a = lm_oracle.fit(tiled, max_iter=20, ad_mode=ad_mode)
    b = lm_oracle.fit(popio.share_y(tiled), max_iter=20, ad_mode=ad_mode)
    for k in ("c_final", "status", "loss_init", "loss_final", "iters"):
        assert np.array_equal(a[k], b[k], equal_nan=True), k


def test_numpy_oracle_reads_shared_target():
    """The numpy scorer and the targets the scipy CPU path fits (interp.y_row,
    interp.tree_view) see the shared row as every expression's target."""
    from oracle import interp

    tiled = _shared_pop(M=12, N=40)
    shared = popio.share_y(tiled)
    c = np.asarray(tiled["c_init"], np.float64)
    assert np.array_equal(interp.loss_pop(shared, c), interp.loss_pop(tiled, c))
    for m in range(12):
        assert np.array_equal(interp.y_row(shared, m), tiled["ym"][m])
        a, b = interp.tree_view(shared, m), interp.tree_view(tiled, m)
        assert all(np.array_equal(x, y) for x, y in zip(a[:4], b[:4])) and a[4] == b[4]
