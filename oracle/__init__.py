"""CPU oracle for the packed-expert routed-MoE path.

TEST INFRASTRUCTURE ONLY. Nothing under `vaayu_amd/` imports, calls or links this
package: only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s CPU-baseline leg
use it, and only as the checker (or, for the baseline, as the thing timed on the host
cores), never as a product path.
"""
