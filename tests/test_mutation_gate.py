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
