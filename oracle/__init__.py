"""CPU oracle of the batched-LM path: test infrastructure, never the product.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package. It holds a C restatement of the reference LM algorithm
(lm_oracle.c), a numpy restatement of the reference scoring interpreter
(interp.py) and the scipy CPU baseline (scipy_pop.py).
"""
