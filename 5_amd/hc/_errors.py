"""Error taxonomy of the hc launch surface (hc/_sim_types.py:62-75)."""

from __future__ import annotations


class SimulatorError(RuntimeError):
    """Runtime failure of a launch (hc/_sim_types.py:62)."""


class LaunchError(SimulatorError):
    """A launch rejected before any execution: binding, dtype, rank or
    geometry (hc/_sim_types.py:66)."""


class ScopeError(SimulatorError):
    """A helper or intrinsic called from the wrong scope (hc/_sim_types.py:70)."""


class PoisonError(SimulatorError):
    """A poison value was observed (hc/_sim_types.py:74)."""


class BackendError(SimulatorError):
    """The gfx950 backend failed after validation (a HIP runtime error, or the
    native library is missing)."""
