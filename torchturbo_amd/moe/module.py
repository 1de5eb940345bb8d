"""Module spec helpers (``src/torchturbo/models/modules/moe/module.py:20-107``)."""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any


@dataclass
class ModuleSpec:
    module: type
    params: dict = field(default_factory=dict)
    submodules: Any = None


def build_module(spec_or_module, *args, **kwargs):
    if spec_or_module is None:
        return None
    if isinstance(spec_or_module, ModuleSpec):
        params = dict(spec_or_module.params)
        params.update(kwargs)
        if spec_or_module.submodules is not None:
            params["submodules"] = spec_or_module.submodules
        return spec_or_module.module(*args, **params)
    if isinstance(spec_or_module, type):
        return spec_or_module(*args, **kwargs)
    return spec_or_module
