"""Which implementations exist for each op, and the order ``auto`` tries them.

Behaviour callers rely on (the reference's ``src/torchturbo/ops/registry.py:35-85``):

* an implementation is known by its ``impl_name``. Registering a name again for
  the same op replaces the earlier spec where it stood; the same name under a
  different op is a ``ValueError``;
* ``list()`` ranks candidates by priority, then device-specific (non-empty
  ``devices``) before device-agnostic, then custom before native, each
  descending; equal candidates keep their registration order.

The table is a dict keyed by ``impl_name``: a dict remembers insertion order and
assigning to an existing key keeps that key's position, which is exactly the
replace-in-place rule, so no separate ordered list is kept.
"""

from __future__ import annotations

from collections.abc import Callable

from ..runtime import TurboDevice
from .base import OpImpl, OpImplKind, OpSpec


def _rank(spec: OpSpec) -> tuple[int, int, int]:
    """Sort key of ``list()`` (larger ranks first)."""
    return (spec.priority, 1 if spec.devices else 0, 1 if spec.kind == OpImplKind.CUSTOM else 0)


class OpRegistry:
    def __init__(self) -> None:
        self._table: dict[str, OpSpec] = {}

    def register(self, spec: OpSpec) -> OpSpec:
        prior = self._table.get(spec.impl_name)
        if prior is not None and prior.op_name != spec.op_name:
            raise ValueError(
                f"impl_name {spec.impl_name!r} cannot serve op {spec.op_name!r}: it is "
                f"already registered for op {prior.op_name!r}."
            )
        self._table[spec.impl_name] = spec
        return spec

    def list(self, spec_filter: Callable[[OpSpec], bool] | None = None) -> list[OpSpec]:
        """Registered specs passing ``spec_filter``, best candidate first."""
        keep = spec_filter or (lambda _spec: True)
        # sorted() is stable, also with reverse=True: ties stay in table order
        return sorted((s for s in self._table.values() if keep(s)), key=_rank, reverse=True)

    def get_by_impl_name(self, impl_name: str) -> OpSpec:
        try:
            return self._table[impl_name]
        except KeyError:
            raise RuntimeError(f"No OpSpec registered for impl_name {impl_name!r}.") from None


registry = OpRegistry()


def register_op(
    *,
    op_name: str,
    impl_name: str,
    kind: OpImplKind,
    priority: int,
    devices: tuple[TurboDevice, ...],
):
    """Class decorator: builds the ``OpSpec`` (validated by its constructor),
    attaches it to the ``OpImpl`` subclass as ``__op_spec__`` and registers it."""
    spec = OpSpec(op_name=op_name, impl_name=impl_name, kind=kind, priority=priority,
                  devices=devices)

    def attach(cls: type[OpImpl]) -> type[OpImpl]:
        cls.__op_spec__ = spec
        registry.register(spec)
        return cls

    return attach


__all__ = ["OpRegistry", "register_op", "registry"]
