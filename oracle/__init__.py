"""CPU oracle for the NKIBench operator set -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference numpy ``forward()`` of every
operator the reference's workspaces optimise, plus the seeded input draws and
the bf16 / relative-L2 helpers of its offline simulators.  Each function cites
the reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the reference that device results are
compared against (or, in bench.py, as the timed host-CPU baseline).  The product (``kda-for-trainium_amd/``) never imports
it and has no CPU fallback.

How each function is pinned (i.e. checked against something other than a
retyping of its own formula) is listed in ``tests/test_oracle.py``; see the
``PINNED_BY`` table in ``oracle.ops``.
"""
from . import inputs, numerics, ops  # noqa: F401
