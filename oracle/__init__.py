"""CPU oracle for the g950 hot path (test infrastructure, never the product).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg import this package; ``compiler_amd`` never does.
"""
