"""Operator boundary: registry, policy-driven dispatcher and the ``ops`` proxy."""

from .base import OpImpl, OpImplKind, OpPolicy, OpSpec
from .dispatcher import OpDispatcher
from .moe import MoEPermutation, get_expert_indices
from .ops import get_ops, get_or_create_ops, ops, reset_ops
from .providers import add_provider_package, iter_provider_modules, remove_provider_package
from .registry import OpRegistry, register_op, registry

__all__ = [
    "MoEPermutation",
    "OpDispatcher",
    "OpImpl",
    "OpImplKind",
    "OpPolicy",
    "OpRegistry",
    "OpSpec",
    "add_provider_package",
    "get_expert_indices",
    "get_ops",
    "get_or_create_ops",
    "iter_provider_modules",
    "ops",
    "register_op",
    "registry",
    "remove_provider_package",
    "reset_ops",
]
