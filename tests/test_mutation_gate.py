"""The mutation gate (oracle/mutation_gate.py) on a few of its mutants, no
GPU: the unmutated oracle passes its pins, and each mutant here -- one from
the solve, one from the elementary functions, one from the AD rules -- makes
tests/test_oracle.py or tests/test_math.py fail. The whole gate (every CPU
mutant) runs as `python oracle/mutation_gate.py`.
"""
from oracle import mutation_gate


def test_mutants_are_killed():
    names = ["pivot-zero-accepted", "cos-quadrant-sign", "exp-coefficient", "adjoint-seed"]
    rows = mutation_gate.run(names)
    assert sorted(r[0] for r in rows) == sorted(names)
    survivors = [r[0] for r in rows if not r[2]]
    assert not survivors, survivors


def test_every_mutant_anchor_is_in_the_sources():
    """Each mutant's edit still finds its text (a source change that moves an
    anchor would make the gate stop at build time)."""
    for name, rel, old, _new, occ, *_rest in mutation_gate.MUTANTS + mutation_gate.DEVICE_MUTANTS:
        if old is None:
            continue
        assert (mutation_gate.REPO / rel).read_text().count(old) > occ, name
