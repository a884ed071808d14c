"""TEST INFRASTRUCTURE ONLY: the CPU oracle for the MoE layer forward.

Nothing in the product package imports this package. Only `tests/`, `__graft_entry__.smoke()`
and `bench.py`'s `cpu_baseline` leg may use it, and only as the checker or the timed CPU
baseline, never as the thing measured or shipped.
"""
