"""``hc.simulator`` launch surface (hc/simulator.py:165-232).

The reference's NumPy/greenlet interpreter is not part of this build (its
semantics are restated as a closed form in the test oracle).  ``launch``
keeps the reference signature and routes by ``target``:

* ``target=hc.gfx950.Gfx950Target(...)`` runs the kernel on gfx950;
* ``target=None`` uses the default target, which is gfx950 when the
  environment sets ``HC_DEFAULT_TARGET=gfx950`` (so an unchanged kernel module
  that calls ``sim.launch(kernel, a, b, c)`` runs on the GPU), and otherwise
  ``SimulatorTarget()``;
* ``SimulatorTarget`` performs the full pre-launch binding and validation
  (so ``LaunchError`` and the zero-size no-op behave as in the reference) and
  then raises ``SimulatorError``: there is no CPU interpreter here.
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
    if os.environ.get("HC_DEFAULT_TARGET", "").lower() in {"gfx950", "amdgpu-gfx950"}:
        from .gfx950 import Gfx950Target

        return Gfx950Target()
    return DEFAULT_TARGET


def launch(fn: Any, *args: Any, target: Any = None, **kwargs: Any) -> None:
    runtime_target = default_target() if target is None else target
    if isinstance(runtime_target, SimulatorTarget):
        prepared = prepare_launch(fn, args, kwargs, runtime_target)
        if prepared.is_empty:
            return
        raise SimulatorError(
            "the host simulator is not part of this build; launch with "
            "target=hc.gfx950.Gfx950Target() (or set HC_DEFAULT_TARGET=gfx950)"
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
