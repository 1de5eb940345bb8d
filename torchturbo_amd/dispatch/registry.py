"""Process-wide operator registry and the ``register_op`` decorator.

Ranking follows ``src/torchturbo/ops/registry.py:35-53``: priority first, then
device-specific over device-agnostic, then custom over native, descending.
Re-registering an ``impl_name`` replaces it in place; the same ``impl_name``
under a different op is an error (``registry.py:14-31``).
"""

from __future__ import annotations

from collections.abc import Callable

from ..runtime import TurboDevice
from .base import OpImpl, OpImplKind, OpSpec


class OpRegistry:
    def __init__(self) -> None:
        self._specs: list[OpSpec] = []
        self._by_impl: dict[str, OpSpec] = {}

    def register(self, spec: OpSpec) -> OpSpec:
        existing = self._by_impl.get(spec.impl_name)
        if existing is not None and existing.op_name != spec.op_name:
            raise ValueError(
                f"OpSpec.impl_name {spec.impl_name!r} is already registered for "
                f"op {existing.op_name!r}."
            )
        for slot, current in enumerate(self._specs):
            if current.impl_name == spec.impl_name:
                self._specs[slot] = spec
                break
        else:
            self._specs.append(spec)
        self._by_impl[spec.impl_name] = spec
        return spec

    def list(self, spec_filter: Callable[[OpSpec], bool] | None = None) -> list[OpSpec]:
        specs = [s for s in self._specs if spec_filter is None or spec_filter(s)]
        specs.sort(
            key=lambda s: (s.priority, bool(s.devices), s.kind == OpImplKind.CUSTOM),
            reverse=True,
        )
        return specs

    def get_by_impl_name(self, impl_name: str) -> OpSpec:
        spec = self._by_impl.get(impl_name)
        if spec is None:
            raise RuntimeError(f"No OpSpec registered for impl_name {impl_name!r}.")
        return spec


registry = OpRegistry()


def register_op(
    *,
    op_name: str,
    impl_name: str,
    kind: OpImplKind,
    priority: int,
    devices: tuple[TurboDevice, ...],
):
    def decorator(cls: type[OpImpl]) -> type[OpImpl]:
        spec = OpSpec(
            op_name=op_name, impl_name=impl_name, kind=kind,
            priority=priority, devices=devices,
        )
        cls.__op_spec__ = spec
        registry.register(spec)
        return cls

    return decorator


__all__ = ["OpRegistry", "register_op", "registry"]
