"""CPU oracle for the hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this package, and only as the checker (or the timed CPU
port).  The device backend never calls it.  See ``oracle.h`` for what each
function restates, the reference lines it follows, and how it is pinned.
"""
