"""CPU oracle for emberserve's fused per-layer ops: TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
this package, and only as the checker (or, for the CPU baseline, as the timed reference
path). The product (`emberserve_amd`) never imports it.

See `ref_ops.py` for the restated functions and how each is pinned.
"""
