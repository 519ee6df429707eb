"""CPU oracle for the GLA hot path: TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
import this package, and only as the checker (or the timed CPU baseline). The product
path (``pallas-kernel_amd/tops``) never imports it and has no CPU fallback.

Every function restates the reference's algorithm in numpy (float64 by default; the layer in
``layer.py`` in float64 torch, for autograd) and cites the reference file:line it follows. How each function is pinned (closed forms, invariants,
autodiff of an independent restatement, finite differences) is recorded in ``gla.py``'s
module docstring and exercised by ``tests/test_oracle.py``.
"""

import importlib

from .gla import *  # noqa: F401,F403

_LAZY = ("layer",        # the GLA layer and its modules, float64 torch
         "simple_gla")   # scalar-gate GLA


def __getattr__(name):
    """``layer`` (which imports torch) and ``simple_gla`` load on first use, so the numpy
    part imports without torch (the CPU baseline's worker processes)."""
    if name in _LAZY:
        return importlib.import_module(f"{__name__}.{name}")
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
