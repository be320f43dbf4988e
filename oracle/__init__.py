"""CPU oracle for the token-sampler path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this package: only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import or run it, and there only as the checker (or as the timed CPU
baseline), never as the thing measured or shipped.
"""
