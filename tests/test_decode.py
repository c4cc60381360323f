"""Host-side decode (co_decode through the C ABI, no GPU): bit-exact round trip
of every program back to the pop.bin nodes, stack depths, K bins, error codes.

The decoded program (cusr_amd/csrc/program.h) folds leaves into operands and
keeps a running value plus spill slots; rebuilding the prefix node list from
it must give back exactly nt / nv / ci, and the constant-rank ranges carried
for forward AD must equal the ranks found in each operand subtree.
"""
import json

import numpy as np
import pytest

from cusr_amd.benchmark import popio
from cusr_amd.kernel import co_inproc as ci
from oracle import lm_oracle
from tests.helpers import GOLDEN, REF_FIX, ref_pop, synth

OP_IDENT = 63


def fields(w):
    w = int(w)
    return dict(fid=w & 63, bin=(w >> 6) & 1, ak=(w >> 7) & 3, ai=(w >> 9) & 15,
                bk=(w >> 13) & 3, bi=(w >> 15) & 15, ts=(w >> 19) & 1, di=(w >> 20) & 15,
                lo=(w >> 24) & 31, mid=(w >> 29) & 31, hi=(w >> 34) & 31, tape=(w >> 39) & 255)


def wfields(a, b):
    """Fields of a wide (general-kernel) instruction, words a and b."""
    a, b = int(a), int(b)
    return dict(fid=a & 63, bin=(a >> 6) & 1, ak=(a >> 7) & 3, ai=(a >> 9) & 255,
                bk=(a >> 17) & 3, bi=(a >> 19) & 255, ts=(a >> 27) & 1, di=(a >> 28) & 255,
                sel=(a >> 36) & 1, sa=(a >> 37) & 1, sb=(a >> 38) & 1, ta=(a >> 39) & 1,
                tb=(a >> 40) & 1, lo=b & 255, mid=(b >> 8) & 255, hi=(b >> 16) & 255,
                tape=(b >> 24) & 0xffffffff)


def instructions(prog, off, n, wide):
    """Field dicts of one expression's program (n words, or 2n for wide)."""
    out = []
    for i in range(n):
        if wide:
            a, b = prog[off + 2 * i], prog[off + 2 * i + 1]
            if a == 0 and b == 0:
                break
            out.append(wfields(a, b))
        else:
            if prog[off + i] == 0:
                break
            out.append(fields(prog[off + i]))
    return out


def rebuild(prog):
    """Prefix node list [(nt, nv, ci)] from a decoded program (field dicts
    or fast-format words), checking ranges."""
    acc = None
    slots = {}

    def operand(kind, idx):
        if kind == 0:
            return acc
        if kind == 1:
            return [(0, float(idx), -1)]
        if kind == 2:
            return [(1, 0.0, idx)]
        return slots.pop(idx)

    def ranks(sub):
        r = [c for t, _, c in sub if t == 1]
        return (min(r), max(r) + 1) if r else None

    for w in prog:
        f = w if isinstance(w, dict) else fields(w)
        a = operand(f["ak"], f["ai"])
        if f["fid"] == OP_IDENT:
            sub = a
        elif f["bin"]:
            b = operand(f["bk"], f["bi"])
            ra, rb = ranks(a), ranks(b)
            if ra:
                assert (f["lo"], f["mid"]) == ra
            if rb:
                assert (f["mid"], f["hi"]) == rb
            sub = [(3, float(f["fid"]), -1)] + a + b
        else:
            ra = ranks(a)
            if ra:
                assert (f["lo"], f["hi"]) == ra
            sub = [(2, float(f["fid"]), -1)] + a
        if f["ts"]:
            assert f["di"] not in slots
            slots[f["di"]] = sub
        else:
            acc = sub
    assert not slots
    return acc


def _pops():
    pops = [ref_pop(n) for n in ("pop1000.bin", "pop_fixture.bin", "pop_fixture_op.bin",
                                  "pop_fixture_stress.bin", "pop_fixture_scale_1e0.bin")]
    pops += [synth("C1", 128, 32)[0], synth("C2", 256, 32)[0], synth("C3", 64, 32)[0],
             synth("C5", 128, 32)[0]]
    return pops


@pytest.mark.parametrize("idx", range(9))
def test_program_round_trip(idx):
    pop = _pops()[idx]
    rc, prog, order, bins, stack = ci.decode(pop)
    assert rc == 0
    off = 0
    for m in range(pop["M"]):
        o, n, _, K = (int(v) for v in pop["metas"][m])
        nins = np.count_nonzero(prog[off:off + n])
        nodes = rebuild(prog[off:off + nins])
        assert [t for t, _, _ in nodes] == pop["nt"][o:o + n].tolist()
        # nv of a CONST node carries nothing (the value lives in c_init)
        nv = pop["nv"][o:o + n].astype(float)
        nv[pop["nt"][o:o + n] == 1] = 0.0
        assert [v for _, v, _ in nodes] == nv.tolist()
        assert [c for _, _, c in nodes] == pop["ci"][o:o + n].tolist()
        off += n


@pytest.mark.parametrize("idx", range(9))
def test_stack_depth_and_k_bins(idx):
    pop = _pops()[idx]
    rc, prog, order, bins, stack = ci.decode(pop)
    assert rc == 0
    K = pop["metas"][:, 3]
    assert np.array_equal(order, np.argsort(K, kind="stable"))
    assert np.array_equal(bins, np.concatenate([[0], np.cumsum(np.bincount(K, minlength=33))]))
    for m in range(pop["M"]):
        o, n, _, _ = (int(v) for v in pop["metas"][m])
        assert stack[m] == popio.stack_depth(pop["nt"][o:o + n])
    orc_rc, orc_stack = lm_oracle.check_pop(pop)
    assert orc_rc == 0 and np.array_equal(orc_stack, stack)


def sethi_ullman(nt):
    """Fewest spill slots an accumulator machine needs for the prefix tree nt
    when each binary operator may run either operand first: a leaf needs no
    instruction; two operands that both need instructions hold one value in a
    slot while the other runs, so equal needs cost one more slot."""
    def walk(i):
        t = nt[i]
        if t <= 1:
            return 0, 1, True
        if t == 2:
            need, size, _ = walk(i + 1)
            return need, size + 1, False
        nl, sl, ll = walk(i + 1)
        nr, sr, lr = walk(i + 1 + sl)
        if not ll and not lr:
            need = nl + 1 if nl == nr else max(nl, nr)
        else:
            need = max(nl, nr)
        return need, sl + sr + 1, False
    return walk(0)[0]


def live_slots(ins):
    """Most spill slots a program holds at once (operands freed before the
    result is stored)."""
    live = peak = 0
    for f in ins:
        live -= (f["ak"] == 3) + (f["bin"] and f["bk"] == 3)
        assert live >= 0
        if f["ts"]:
            live += 1
            peak = max(peak, live)
    assert live == 0
    return peak


@pytest.mark.parametrize("idx", range(9))
def test_spill_slots_are_minimal(idx):
    """Operands run in Sethi-Ullman order: every program holds no more spill
    slots at once than the tree's minimum (the LDS each wavefront reserves)."""
    pop = _pops()[idx]
    rc, prog, order, bins, stack = ci.decode(pop)
    assert rc == 0
    off = 0
    for m in range(pop["M"]):
        o, n, _, _ = (int(v) for v in pop["metas"][m])
        ins = instructions(prog, off, n, False)
        assert live_slots(ins) == sethi_ullman(pop["nt"][o:o + n].tolist())
        off += n


def test_sethi_ullman_order_cases():
    """Hand-made trees: two leaf pairs need one slot in either order; a full
    tree of depth 3 needs 2; when the left operand needs more slots it runs
    first, so the tree needs 1 where the right-first order needs 2."""
    pair = [3, 0, 0]                       # x0 + x0
    two_pairs = [3] + pair + pair          # (x0 + x0) + (x0 + x0): 1 slot in either order
    full = [3] + two_pairs + two_pairs     # full depth-3 tree: 2 slots
    lean = [3] + two_pairs + pair          # right operand first would hold 2
    trees = [(t, [1.0 if x == 3 else 0.0 for x in t], [-1] * len(t), np.zeros(0))
             for t in (two_pairs, full, lean)]
    pop = popio.build_pop(trees, np.zeros((4, 1)), np.zeros((3, 4)))
    rc, prog, order, bins, stack = ci.decode(pop)
    assert rc == 0
    got = []
    off = 0
    for m in range(pop["M"]):
        o, n, _, _ = (int(v) for v in pop["metas"][m])
        got.append(live_slots(instructions(prog, off, n, False)))
        off += n
    assert got == [1, 2, 1]
    assert [sethi_ullman(t[0]) for t in trees] == [1, 2, 1]


# flat-branch operators (the select rule): MAX, MIN, LT, GT, LE, GE, PDIV, CEXP
SELECT_OPS = {8, 9, 10, 11, 12, 13, 32, 33}


@pytest.mark.parametrize("idx", range(9))
def test_ad_flags_and_tape_slots(idx):
    """Per-instruction AD fields (bits 47..51): reverse-AD tape slots are dense
    and in execution order; a side has one exactly when its partial is read
    (not a variable) and not exactly +-1 (ADD, SUB, the identity); forward-AD
    scale flags never point at an empty rank range."""
    pop = _pops()[idx]
    rc, prog, order, bins, stack = ci.decode(pop)
    assert rc == 0
    for m in range(pop["M"]):
        o, n, _, _ = (int(v) for v in pop["metas"][m])
        nxt = 0
        for w in prog[o:o + n]:
            w = int(w)
            if w == 0:
                break
            f = fields(w)
            sel, sa, sb, ta, tb = ((w >> b) & 1 for b in (47, 48, 49, 50, 51))
            assert f["tape"] == nxt
            nxt += ta + tb
            unit = f["fid"] in (1, 2) or f["fid"] == OP_IDENT
            assert ta == int(f["ak"] != 1 and not unit)
            assert tb == int(bool(f["bin"]) and f["bk"] != 1 and not unit)
            assert sel == int(f["fid"] in SELECT_OPS)
            if sa:
                assert f["mid"] > f["lo"] and f["fid"] not in (1, 2, OP_IDENT)
            if sb:
                assert f["bin"] and f["hi"] > f["mid"] and f["fid"] != 1
            # a scaled range is exactly a non-empty one whose partial is not 1
            if f["bin"]:
                assert sa == int(f["mid"] > f["lo"] and f["fid"] not in (1, 2))
                assert sb == int(f["hi"] > f["mid"] and f["fid"] != 1)


def test_reference_header_stats():
    """pop1000.bin header matches the reference golden manifest."""
    pop = ref_pop("pop1000.bin")
    man = json.loads((REF_FIX / "golden_manifest.json").read_text())
    h = man["variants"]["ad"]["pop1000"]["header"]
    for k_ref, k in (("M_prob", "M"), ("total_nodes", "total_nodes"), ("total_c", "total_c"),
                     ("N", "N"), ("n_vars", "n_vars"), ("K_max", "K_max"),
                     ("max_stack", "max_stack")):
        assert pop[k] == h[k_ref]
    size = (REF_FIX / "pop1000.bin").stat().st_size
    assert size == popio.pop_bytes(pop["M"], pop["total_nodes"], pop["total_c"], pop["N"],
                                   pop["n_vars"]) == 4273688


def _tiny():
    # x0 * c0 + c1  ->  prefix [ADD, MUL, x0, c0, c1]
    trees = [([3, 3, 0, 1, 1], [1, 3, 0, 0, 0], [-1, -1, -1, 0, 1], [1.0, 2.0])]
    xs = np.linspace(-1, 1, 8).reshape(8, 1)
    return popio.build_pop(trees, xs, np.zeros((1, 8)))


def _code(pop):
    return ci.decode(pop)[0]


def test_error_codes():
    good = _tiny()
    assert _code(good) == 0
    bad = dict(good); bad["total_c"] = 3
    assert _code(bad) == ci.CO_ERR_SUM_C
    bad = dict(good); bad["total_nodes"] = 6
    assert _code(bad) == ci.CO_ERR_SUM_NODES
    bad = dict(good); bad["nv"] = good["nv"].copy(); bad["nv"][0] = 29.0   # unknown op id
    assert _code(bad) == ci.CO_ERR_PROGRAM
    bad = dict(good); bad["nt"] = good["nt"].copy(); bad["nt"][0] = 4      # ternary node
    assert _code(bad) == ci.CO_ERR_PROGRAM
    bad = dict(good); bad["ci"] = good["ci"].copy(); bad["ci"][3] = 1      # ranks out of order
    bad["ci"][4] = 0
    assert _code(bad) == ci.CO_ERR_PROGRAM
    bad = dict(good); bad["nv"] = good["nv"].copy(); bad["nv"][2] = 1.0    # var index >= n_vars
    assert _code(bad) == ci.CO_ERR_PROGRAM
    bad = dict(good); bad["nt"] = good["nt"].copy(); bad["nt"][1] = 2      # MUL as unary: stack
    assert _code(bad) == ci.CO_ERR_PROGRAM
    # header bounds, checked first like co_lib.cu:211-212: K_max 32 and
    # max_stack 64 are the reference's; n_vars up to 255
    for key, ok, beyond in (("K_max", 32, 33), ("max_stack", 64, 65), ("n_vars", 255, 256)):
        bad = dict(good); bad[key] = beyond
        assert _code(bad) == ci.CO_ERR_BOUNDS, key
        fine = dict(good); fine[key] = ok
        assert _code(fine) in (0, ci.CO_ERR_PROGRAM), key   # n_vars changes nothing valid


def _sum_tree(K):
    """c0 + c1 + ... + c_{K-1} + x0 as a left spine: stack 2, K constants."""
    nt = [3] * K + [0] + [1] * K
    nv = [1.0] * K + [0.0] * (K + 1)
    cis = [-1] * (K + 1) + list(range(K))
    return nt, nv, cis


def test_bounds_per_expression():
    """K 17..32 decodes (general kernel), K 33 is refused even when the header
    understates it; a value stack of 64 decodes, 65 is refused."""
    for K, want in ((17, 0), (28, 0), (32, 0), (33, ci.CO_ERR_BOUNDS)):
        nt, nv, cis = _sum_tree(K)
        pop = popio.build_pop([(nt, nv, cis, np.zeros(K))], np.zeros((4, 1)), np.zeros((1, 4)))
        assert pop["K_max"] == K
        assert _code(pop) == want, K
        under = dict(pop); under["K_max"] = 8
        assert _code(under) == want, K
    from tests.general_pops import deep_tree
    rng = np.random.default_rng(0)
    for S, want in ((63, 0), (64, ci.CO_ERR_BOUNDS)):    # stack S + 1
        nt, nv, cis, K = deep_tree(rng, S, 2, 8)
        pop = popio.build_pop([(nt, nv, cis, np.zeros(K))], np.zeros((4, 2)), np.zeros((1, 4)))
        assert pop["max_stack"] == S + 1
        under = dict(pop); under["max_stack"] = 10
        assert _code(under) == want, S


@pytest.mark.parametrize("kind", ["highk", "deep", "long", "wide", "mixed"])
def test_general_programs_round_trip_and_route(kind):
    """Expressions outside co_fast_path get wide programs (two words per
    instruction, laid out after the previous expression's words) that
    rebuild to their nodes exactly; the route is co_fast_path's answer."""
    from tests.general_pops import general_pop
    pop, _ = general_pop(kind, 24, 64)
    rc, prog, order, bins, stack, poff, route = ci.decode(pop, full=True)
    assert rc == 0
    D = pop["n_vars"]
    off = 0
    for m in range(pop["M"]):
        o, n, _, K = (int(v) for v in pop["metas"][m])
        fast = ci.co_fast_path(K, int(stack[m]), n, D)
        assert route[m] == (0 if fast else 1)
        assert poff[m] == off
        ins = instructions(prog, off, n, not fast)
        nodes = rebuild(ins)
        assert [t for t, _, _ in nodes] == pop["nt"][o:o + n].tolist()
        nv = pop["nv"][o:o + n].astype(float)
        nv[pop["nt"][o:o + n] == 1] = 0.0
        assert [v for _, v, _ in nodes] == nv.tolist()
        assert [c for _, _, c in nodes] == pop["ci"][o:o + n].tolist()
        if not fast:
            # the wide fields: dense tape slots and the AD flags of the fast format
            nxt = 0
            for f in ins:
                assert f["tape"] == nxt
                nxt += f["ta"] + f["tb"]
                unit = f["fid"] in (1, 2) or f["fid"] == OP_IDENT
                assert f["ta"] == int(f["ak"] != 1 and not unit)
                assert f["sel"] == int(f["fid"] in SELECT_OPS)
                if f["bin"]:
                    assert f["sa"] == int(f["mid"] > f["lo"] and f["fid"] not in (1, 2))
                    assert f["sb"] == int(f["hi"] > f["mid"] and f["fid"] != 1)
        off += n if fast else 2 * n
    if kind != "mixed":
        assert route.all()
    else:
        assert 0 < route.sum() < pop["M"]


@pytest.mark.parametrize("variant,order", [("ad", 0), ("fd", 1)])
def test_library_exports_every_header_symbol(variant, order):
    import ctypes
    import re
    hdr = (GOLDEN.parents[1] / "include" / "cusr_co.h").read_text()
    names = set(re.findall(r"^\s*(?:int|void)\s+(co_\w+)\s*\(", hdr, re.M))
    assert names == set(ci.EXPORTED)
    lib = ci.load_library(variant)
    for n in names:
        assert hasattr(lib, n), n
    o = ci.CoOptions()
    lib.co_options_default(ctypes.byref(o))          # host-only, no device needed
    assert o.struct_size == ctypes.sizeof(ci.CoOptions) and o.lm_order == order
