"""Operator metadata: policy, kind, spec and the provider base class.

Same contract as the reference's ``src/torchturbo/ops/base.py:11-60``:
``OpSpec`` validates its names, reserves the policy names, and normalises
``priority``/``devices``; ``OpImpl.available()`` must not raise.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from dataclasses import dataclass
from enum import Enum
from typing import Any, ClassVar

from ..runtime import TurboDevice


class OpPolicy(str, Enum):
    AUTO = "auto"
    NATIVE = "native"
    CUSTOM = "custom"

    def __str__(self) -> str:
        return self.value


class OpImplKind(str, Enum):
    NATIVE = "native"
    CUSTOM = "custom"

    def __str__(self) -> str:
        return self.value


@dataclass(frozen=True)
class OpSpec:
    op_name: str
    impl_name: str
    kind: OpImplKind = OpImplKind.NATIVE
    priority: int = 0
    devices: tuple[TurboDevice, ...] = ()

    def __post_init__(self) -> None:
        if not self.op_name:
            raise ValueError("OpSpec.op_name must be set.")
        if not self.impl_name:
            raise ValueError("OpSpec.impl_name must be set.")
        if self.impl_name in {item.value for item in OpPolicy}:
            raise ValueError(
                f"OpSpec.impl_name cannot be a reserved policy name: {self.impl_name!r}."
            )
        if not isinstance(self.kind, OpImplKind):
            raise TypeError("OpSpec.kind must be an OpImplKind.")
        object.__setattr__(self, "priority", int(self.priority))
        object.__setattr__(self, "devices", tuple(self.devices))


class OpImpl(ABC):
    __op_spec__: ClassVar[OpSpec | None] = None

    @classmethod
    def op_spec(cls) -> OpSpec:
        spec = cls.__op_spec__
        if spec is None:
            raise RuntimeError(f"{cls.__name__} is missing op spec metadata.")
        return spec

    def available(self) -> bool:
        return True

    @abstractmethod
    def __call__(self, *args: Any, **kwargs: Any):
        raise NotImplementedError


__all__ = ["OpImpl", "OpImplKind", "OpPolicy", "OpSpec"]
