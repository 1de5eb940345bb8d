"""Process-wide dispatcher singleton and the ``ops`` proxy.

Same reuse rules as ``src/torchturbo/ops/ops.py:15-80``: a second request
must match device, policy and overrides, otherwise ``RuntimeError``.
"""

from __future__ import annotations

from collections.abc import Mapping

from ..runtime import DeviceRuntime
from .base import OpPolicy
from .dispatcher import OpDispatcher
from .registry import registry

_OPS: OpDispatcher | None = None


def get_or_create_ops(
    *,
    device_runtime: DeviceRuntime,
    default_policy: OpPolicy = OpPolicy.AUTO,
    overrides: Mapping[str, str] | None = None,
) -> OpDispatcher:
    global _OPS
    if not isinstance(default_policy, OpPolicy):
        raise TypeError("default_policy must be an OpPolicy.")
    requested = dict(overrides or {})
    if _OPS is None:
        _OPS = OpDispatcher(device_runtime=device_runtime, registry=registry,
                            default_policy=default_policy, overrides=requested)
        return _OPS
    conflicts = []
    if _OPS.device_runtime.turbo_device != device_runtime.turbo_device:
        conflicts.append(f"device={_OPS.device_runtime.turbo_device.value!r} vs "
                         f"{device_runtime.turbo_device.value!r}")
    if _OPS.default_policy != default_policy:
        conflicts.append(f"policy={_OPS.default_policy.value!r} vs {default_policy.value!r}")
    if _OPS.overrides != requested:
        conflicts.append(f"overrides={_OPS.overrides!r} vs {requested!r}")
    if conflicts:
        raise RuntimeError(
            "Ops dispatcher is already configured for this process with an "
            "incompatible configuration (" + ", ".join(conflicts) + ")."
        )
    return _OPS


def get_ops() -> OpDispatcher:
    if _OPS is None:
        raise RuntimeError("Ops dispatcher is not configured. Call get_or_create_ops().")
    return _OPS


def reset_ops() -> None:
    """Drop the process dispatcher (tests and benchmarks switch devices)."""
    global _OPS
    _OPS = None


class _OpsProxy:
    def __getattr__(self, name: str):
        return getattr(get_ops(), name)

    def __repr__(self) -> str:
        return "<ops proxy>"


ops = _OpsProxy()

__all__ = ["get_or_create_ops", "get_ops", "ops", "reset_ops"]
