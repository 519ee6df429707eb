"""CPU oracle for the GLA hot path: TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
import this package, and only as the checker (or the timed CPU baseline). The product
path (``pallas-kernel_amd/tops``) never imports it and has no CPU fallback.

Every function restates the reference's algorithm in numpy (float64 by default; the layer in
``layer.py`` in float64 torch, for autograd) and cites the reference file:line it follows. How each function is pinned (closed forms, invariants,
autodiff of an independent restatement, finite differences) is recorded in ``gla.py``'s
module docstring and exercised by ``tests/test_oracle.py``.
"""

from .gla import *  # noqa: F401,F403
from . import layer  # noqa: F401  (the GLA layer and its modules, float64 torch)
from . import simple_gla  # noqa: F401  (scalar-gate GLA)
