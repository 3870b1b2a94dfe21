"""``hc.simulator`` launch surface (hc/simulator.py:165-232).

The reference's NumPy/greenlet interpreter is not part of this build (its
semantics are restated as a closed form in the test oracle).  ``launch``
keeps the reference signature and routes by ``target``:

* ``target=None`` uses the default target: gfx950 when the native library is
  built and a gfx950 GPU is visible, so the reference's unchanged
  ``sim.launch(kernel, a, b, c)`` runs on the GPU
  (examples/amdgpu_gfx11_wmma_matmul.py:338-348); otherwise
  ``SimulatorTarget()``.  ``HC_DEFAULT_TARGET=gfx950`` or ``=simulator``
  forces the choice;
* ``target=hc.gfx950.Gfx950Target(...)`` runs the kernel on gfx950;
* an explicit ``SimulatorTarget`` performs the full pre-launch binding and
  validation (so ``LaunchError`` and the zero-size no-op behave as in the
  reference) and then raises ``SimulatorError``: there is no CPU
  interpreter here.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Any

from ._errors import LaunchError, PoisonError, ScopeError, SimulatorError
from ._launch import default_group_shape, prepare_launch


@dataclass(frozen=True)
class SimulatorTarget:
    """Launch-policy knobs of the reference simulator (hc/simulator.py:60-75)."""

    max_group_size: int | None = None

    def choose_group_shape(self, work_shape: tuple[int, ...], subgroup_size: int | None) -> tuple[int, ...]:
        return default_group_shape(work_shape, subgroup_size)


DEFAULT_TARGET = SimulatorTarget()


def default_target() -> Any:
    """The target of ``launch(..., target=None)``."""
    choice = os.environ.get("HC_DEFAULT_TARGET", "").strip().lower()
    if choice in {"simulator", "host"}:
        return DEFAULT_TARGET
    from . import gfx950

    if choice in {"gfx950", "amdgpu-gfx950"} or (not choice and gfx950.device_available()):
        return gfx950.Gfx950Target()
    return DEFAULT_TARGET


def launch(fn: Any, *args: Any, target: Any = None, **kwargs: Any) -> None:
    runtime_target = default_target() if target is None else target
    if isinstance(runtime_target, SimulatorTarget):
        prepared = prepare_launch(fn, args, kwargs, runtime_target)
        if prepared.is_empty:
            return
        raise SimulatorError(
            "the host simulator is not part of this build; launch on a gfx950 GPU "
            "(target=None picks it when one is visible, or target=hc.gfx950.Gfx950Target())"
        )
    from . import gfx950

    if not isinstance(runtime_target, gfx950.Gfx950Target):
        raise LaunchError(f"unsupported launch target {runtime_target!r}")
    gfx950.launch(fn, *args, target=runtime_target, **kwargs)


run = launch

__all__ = [
    "DEFAULT_TARGET",
    "LaunchError",
    "PoisonError",
    "ScopeError",
    "SimulatorError",
    "SimulatorTarget",
    "launch",
    "run",
]
