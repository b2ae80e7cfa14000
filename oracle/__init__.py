"""CPU oracle for the state codec and FP4 decode: test infrastructure only.

Only `tests/`, `__graft_entry__.smoke()` and the CPU-baseline leg of
`bench.py` load this package.  It is the checker, never the thing shipped.
"""
