"""CPU oracle for the Marlin hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker (or the timed CPU reference path), never as the product.
The product path (marlin_v100_amd) never imports it.

Every function restates the reference's algorithm and cites the reference file:line it
follows.  Pinning of each function (golden vectors, closed forms, invariants) is listed in
tests/test_oracle.py.
"""
from .marlin_ref import *  # noqa: F401,F403
