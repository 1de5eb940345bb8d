"""The process-wide dispatcher and the ``ops`` proxy that forwards to it.

A process has one dispatcher (the reference's ``src/torchturbo/ops/ops.py:15-80``):
the first ``get_or_create_ops`` call creates it; later calls get the same
object back only when they ask for the same device, default policy and per-op
overrides, and otherwise fail with ``RuntimeError`` naming what differs.
"""

from __future__ import annotations

from collections.abc import Mapping

from ..runtime import DeviceRuntime
from .base import OpPolicy
from .dispatcher import OpDispatcher
from .registry import registry

_OPS: OpDispatcher | None = None


def _differences(current: OpDispatcher, device_runtime: DeviceRuntime, policy: OpPolicy,
                 overrides: dict[str, str]) -> list[str]:
    """``name=installed vs requested`` for every setting that does not match."""
    settings = (
        ("device", current.device_runtime.turbo_device.value, device_runtime.turbo_device.value),
        ("policy", current.default_policy.value, policy.value),
        ("overrides", current.overrides, overrides),
    )
    return [f"{name}={have!r} vs {want!r}" for name, have, want in settings if have != want]


def get_or_create_ops(
    *,
    device_runtime: DeviceRuntime,
    default_policy: OpPolicy = OpPolicy.AUTO,
    overrides: Mapping[str, str] | None = None,
) -> OpDispatcher:
    """The process dispatcher, created on first use with these settings."""
    global _OPS
    if not isinstance(default_policy, OpPolicy):
        raise TypeError("default_policy must be an OpPolicy.")
    wanted = dict(overrides or {})
    if _OPS is None:
        _OPS = OpDispatcher(device_runtime=device_runtime, registry=registry,
                            default_policy=default_policy, overrides=wanted)
        return _OPS
    mismatch = _differences(_OPS, device_runtime, default_policy, wanted)
    if mismatch:
        raise RuntimeError(
            "This process already has an ops dispatcher, with an incompatible "
            "configuration: " + "; ".join(mismatch) + "."
        )
    return _OPS


def get_ops() -> OpDispatcher:
    """The installed dispatcher; ``RuntimeError`` before ``get_or_create_ops``."""
    if _OPS is None:
        raise RuntimeError("No ops dispatcher is configured yet: call get_or_create_ops() first.")
    return _OPS


def reset_ops() -> None:
    """Forget the process dispatcher (tests and benchmarks switch devices)."""
    global _OPS
    _OPS = None


class _OpsProxy:
    """``ops.<facade>(...)`` resolves the dispatcher at call time."""

    def __getattr__(self, name: str):
        return getattr(get_ops(), name)

    def __repr__(self) -> str:
        return "<ops proxy>"


ops = _OpsProxy()

__all__ = ["get_or_create_ops", "get_ops", "ops", "reset_ops"]
