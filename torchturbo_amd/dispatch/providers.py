"""Provider-module discovery.

As in the reference (``src/torchturbo/ops/providers/__init__.py:9-32``), every
non-package module of a provider package whose dotted path has no
``_``-prefixed component is imported so its ``@register_op`` decorators run.

The product ships one provider package: ``torchturbo_amd.providers.hip``
(GPU only). It ships no native/CPU provider: the pure-PyTorch restatement of
the reference's native providers is test infrastructure and is attached by
the test-suite with :func:`add_provider_package`.
"""

from __future__ import annotations

from importlib import import_module
from pkgutil import walk_packages

from ..runtime import TurboDevice

_BUILTIN: dict[TurboDevice, tuple[str, ...]] = {
    TurboDevice.CUDA: ("torchturbo_amd.providers.hip",),
    TurboDevice.CPU: (),
    TurboDevice.NPU: (),
}
_EXTRA: list[tuple[str, tuple[TurboDevice, ...]]] = []


def _iter_package_modules(package_name: str) -> tuple[str, ...]:
    package = import_module(package_name)
    if not hasattr(package, "__path__"):
        return (package_name,)
    modules = []
    for info in walk_packages(package.__path__, f"{package.__name__}."):
        relative = info.name[len(package.__name__) + 1:]
        if info.ispkg or any(part.startswith("_") for part in relative.split(".")):
            continue
        modules.append(info.name)
    return tuple(sorted(modules))


def add_provider_package(package_name: str, devices: tuple[TurboDevice, ...] = ()) -> None:
    """Discover ``package_name`` for ``devices`` (all devices when empty)."""
    entry = (package_name, tuple(devices))
    if entry not in _EXTRA:
        _EXTRA.append(entry)


def remove_provider_package(package_name: str) -> None:
    _EXTRA[:] = [e for e in _EXTRA if e[0] != package_name]


def iter_provider_modules(device: TurboDevice) -> tuple[str, ...]:
    if device not in _BUILTIN:
        raise ValueError(f"Unsupported op provider device: {device!r}.")
    modules: list[str] = []
    for package_name, devices in _EXTRA:
        if not devices or device in devices:
            modules.extend(_iter_package_modules(package_name))
    for package_name in _BUILTIN[device]:
        modules.extend(_iter_package_modules(package_name))
    return tuple(modules)


__all__ = ["add_provider_package", "iter_provider_modules", "remove_provider_package"]
