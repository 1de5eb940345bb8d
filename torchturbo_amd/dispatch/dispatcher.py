"""Operator dispatcher with the reference's selection policy and MoE facades.

Selection semantics follow ``src/torchturbo/ops/dispatcher.py:108-293``:

* ``_configure`` resolves every registered op for the runtime's device and
  records (does not raise on) unresolved ones; an invalid config override
  raises ``RuntimeError`` at construction;
* an explicit ``impl=`` or an override never falls back (``148-160``);
* ``native`` / ``custom`` policies filter by kind and never cross over;
  ``auto`` walks the ranked candidates past unavailable ones (``162-186``);
* the first available candidate per (op, device, impl) is cached.

Facades (``moe_permutation`` ``530-590``, ``moe_unpermutation`` ``592-637``,
``moe_sort_chunks`` ``639-660``, ``grouped_matmul`` ``311-327``,
``swiglu`` ``365-375``, ``gated_activation`` ``347-363``) keep the reference's
argument names and validation errors; any other registered op name is
reachable through ``__getattr__`` (``662-671``).
"""

from __future__ import annotations

import importlib
import logging
from collections.abc import Mapping
from dataclasses import dataclass
from types import ModuleType
from typing import Any

import torch

from ..runtime import DeviceRuntime, TurboDevice
from .base import OpImpl, OpImplKind, OpPolicy, OpSpec
from .moe import MoEPermutation, get_expert_indices
from .providers import iter_provider_modules
from .registry import OpRegistry

logger = logging.getLogger("torchturbo_amd")


@dataclass(frozen=True)
class _Candidate:
    impl: OpImpl
    spec: OpSpec
    fallback: bool


class OpDispatcher:
    def __init__(
        self,
        *,
        device_runtime: DeviceRuntime,
        registry: OpRegistry,
        default_policy: OpPolicy = OpPolicy.AUTO,
        overrides: Mapping[str, str] | None = None,
    ) -> None:
        if not isinstance(default_policy, OpPolicy):
            raise TypeError("default_policy must be an OpPolicy.")
        self.registry = registry
        self._device_runtime = device_runtime
        self._default_policy = default_policy
        self._overrides = dict(overrides or {})
        if any(not isinstance(k, str) or not isinstance(v, str)
               for k, v in self._overrides.items()):
            raise TypeError("overrides must map op names to implementation names.")
        self._impls: dict[str, OpImpl] = {}
        self._impl_classes: dict[str, type[OpImpl]] = {}
        self._cache: dict[tuple[str, str, str | None], _Candidate] = {}
        self._unresolved_ops: dict[str, str] = {}
        self._configure()

    @property
    def device_runtime(self) -> DeviceRuntime:
        return self._device_runtime

    @property
    def default_policy(self) -> OpPolicy:
        return self._default_policy

    @property
    def overrides(self) -> dict[str, str]:
        return dict(self._overrides)

    @property
    def unresolved_ops(self) -> dict[str, str]:
        return dict(self._unresolved_ops)

    # -- provider indexing -------------------------------------------------
    @staticmethod
    def _index_provider_module(module: ModuleType, classes: dict[str, type[OpImpl]]) -> None:
        for value in module.__dict__.values():
            if not isinstance(value, type) or value.__module__ != module.__name__:
                continue
            if not issubclass(value, OpImpl) or value is OpImpl:
                continue
            try:
                spec = value.op_spec()
            except RuntimeError:
                continue
            existing = classes.get(spec.impl_name)
            if existing is not None and existing is not value:
                raise ValueError(
                    f"Op implementation {spec.impl_name!r} is defined by both "
                    f"{existing.__module__}.{existing.__qualname__} and "
                    f"{value.__module__}.{value.__qualname__}."
                )
            classes[spec.impl_name] = value

    def _configure(self) -> None:
        device = self._device_runtime.turbo_device
        classes: dict[str, type[OpImpl]] = {}
        for name in iter_provider_modules(device):
            self._index_provider_module(importlib.import_module(name), classes)
        self._impl_classes = classes
        specs = self.registry.list(lambda s: not s.devices or device in s.devices)
        op_names = {s.op_name for s in specs if s.impl_name in classes}
        op_names.update(self._overrides)
        for op_name in sorted(op_names):
            override = self._overrides.get(op_name)
            try:
                self._candidate_impl(op_name, device, impl=override)
            except RuntimeError as exc:
                if override is not None:
                    raise RuntimeError(
                        f"Invalid override for op {op_name!r}: {override!r}. {exc}"
                    ) from exc
                self._unresolved_ops[op_name] = str(exc)

    # -- selection ---------------------------------------------------------
    def _candidate_impl(self, op_name: str, device: TurboDevice, impl: str | None = None) -> OpImpl:
        key = (op_name, device.value, impl)
        cached = self._cache.get(key)
        if cached is not None:
            return cached.impl
        if impl is not None:
            spec = self.registry.get_by_impl_name(impl)
            if spec.op_name != op_name:
                raise RuntimeError(
                    f"Implementation {impl!r} is registered for op {spec.op_name!r}, "
                    f"not {op_name!r}."
                )
            if spec.devices and device not in spec.devices:
                raise RuntimeError(
                    f"Implementation {impl!r} for op {op_name!r} does not support "
                    f"device={device.value}."
                )
            specs = [spec]
        else:
            policy = self._default_policy

            def matches(spec: OpSpec) -> bool:
                if spec.op_name != op_name or spec.impl_name not in self._impl_classes:
                    return False
                if spec.devices and device not in spec.devices:
                    return False
                if policy == OpPolicy.NATIVE:
                    return spec.kind == OpImplKind.NATIVE
                if policy == OpPolicy.CUSTOM:
                    return spec.kind == OpImplKind.CUSTOM
                return True

            specs = self.registry.list(matches)

        unavailable: list[str] = []
        for spec in specs:
            impl_obj = self._load_impl(spec)
            if not impl_obj.available():
                unavailable.append(spec.impl_name)
                continue
            self._cache[key] = _Candidate(impl_obj, spec, bool(unavailable))
            return impl_obj
        detail = f" (unavailable={unavailable})" if unavailable else ""
        selected = f"policy={self._default_policy.value}" if impl is None else f"impl={impl}"
        raise RuntimeError(
            f"No implementation for op={op_name!r}, device={device.value}, {selected}{detail}."
        )

    def _load_impl(self, spec: OpSpec) -> OpImpl:
        impl = self._impls.get(spec.impl_name)
        if impl is not None:
            return impl
        cls = self._impl_classes.get(spec.impl_name)
        if cls is None:
            raise RuntimeError(f"No OpImpl class registered for impl_name {spec.impl_name!r}.")
        impl = cls()
        self._impls[spec.impl_name] = impl
        return impl

    def selected_impl_name(self, op_name: str) -> str:
        """Name of the implementation the dispatcher would run for ``op_name``."""
        device = self._device_runtime.turbo_device
        override = self._overrides.get(op_name)
        self._candidate_impl(op_name, device, impl=override)
        return self._cache[(op_name, device.value, override)].spec.impl_name

    def log_ops_selection(self) -> str:
        """Log (and return) the op → implementation table (``dispatcher.py:213-277``)."""
        rows = []
        chosen = {op: c for (op, _, impl), c in self._cache.items()
                  if impl == self._overrides.get(op)}
        for op_name in sorted(set(chosen) | set(self._unresolved_ops)):
            cand = chosen.get(op_name)
            if cand is None:
                rows.append((op_name, "-", "-", "-", "unavailable"))
                continue
            status = ("overridden" if op_name in self._overrides
                      else "fallback" if cand.fallback else "selected")
            rows.append((op_name, cand.spec.impl_name, cand.spec.kind.value,
                         str(cand.spec.priority), status))
        if not rows:
            rows.append(("<no registered ops>", "-", "-", "-", "-"))
        headers = ("Op", "Implementation", "Kind", "Priority", "Status")
        widths = [max(len(h), *(len(r[i]) for r in rows)) + 2 for i, h in enumerate(headers)]
        fmt = lambda r: " ".join(f"{v:<{w}}" for v, w in zip(r, widths)).rstrip()  # noqa: E731
        sep = "-" * len(fmt(headers))
        lines = [sep, fmt(headers), sep, *(fmt(r) for r in rows), sep]
        details = [f"  {op}: {msg}" for op, msg in sorted(self._unresolved_ops.items())]
        if details:
            lines += ["", "Unavailable details:", *details]
        text = "\n".join(lines)
        logger.info("ops selection (device=%s, policy=%s):\n%s",
                    self._device_runtime.device.type, self._default_policy.value, text)
        return text

    def _dispatch(self, op_name: str, *args: Any, impl: str | None = None, **kwargs: Any):
        device = self._device_runtime.turbo_device
        selected = impl if impl is not None else self._overrides.get(op_name)
        return self._candidate_impl(op_name, device, impl=selected)(*args, **kwargs)

    # -- MoE facades -------------------------------------------------------
    def grouped_matmul(self, x, weight, group_list, *, trans_b: bool = False,
                       impl: str | None = None):
        """``Y[s_e:s_e+n_e] = X[s_e:s_e+n_e] @ W[e]`` (``W[e].T`` with ``trans_b``)."""
        return self._dispatch("grouped_matmul", x, weight, group_list, trans_b=trans_b, impl=impl)

    def gated_activation(self, x, *, activation_func, limit: float = 0.0,
                         clamp_gate_after_activation: bool = False, impl: str | None = None):
        return self._dispatch(
            "gated_activation", x, activation_func=activation_func, limit=limit,
            clamp_gate_after_activation=clamp_gate_after_activation, impl=impl,
        )

    def swiglu(self, x, *, impl: str | None = None):
        return self._dispatch("swiglu", x, impl=impl)

    def moe_permutation(
        self,
        tokens: torch.Tensor,
        routing_map: torch.Tensor,
        probs: torch.Tensor | None = None,
        num_out_tokens: int | None = None,
        expert_indices: torch.Tensor | None = None,
        *,
        impl: str | None = None,
    ) -> MoEPermutation:
        """Duplicate and group token assignments by expert, without weighting.

        Rows are ordered by expert id, then source token id; selected routes
        are kept even when their weight is zero. ``num_out_tokens`` must equal
        ``num_tokens * topk`` (token dropping is unsupported).
        """
        if expert_indices is None:
            expert_indices = get_expert_indices(routing_map)
        expected = expert_indices.numel()
        if num_out_tokens is not None and num_out_tokens != expected:
            raise ValueError(
                "num_out_tokens must equal num_tokens * topk; token dropping is unsupported."
            )
        return self._dispatch(
            "moe_permutation", tokens, routing_map, probs=probs,
            num_out_tokens=expected, expert_indices=expert_indices, impl=impl,
        )

    def moe_unpermutation(
        self,
        permutation: MoEPermutation,
        restore_shape: torch.Size,
        probs: torch.Tensor | None = None,
        *,
        impl: str | None = None,
    ) -> torch.Tensor:
        """``out[i] = sum_j tokens[row_indices[i, j]] (* probs[i, expert_indices[i, j]])``."""
        return self._dispatch("moe_unpermutation", permutation, restore_shape,
                              probs=probs, impl=impl)

    def moe_sort_chunks(
        self,
        input: torch.Tensor,
        split_sizes: torch.Tensor,
        sorted_idxs: torch.Tensor,
        probs: torch.Tensor | None = None,
        *,
        impl: str | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor | None]:
        """Reorder row chunks; metadata must live on the input device."""
        if split_sizes.device != input.device or sorted_idxs.device != input.device:
            raise ValueError(
                "Chunk sorting requires split_sizes and sorted_idxs on the input device."
            )
        return self._dispatch("moe_sort_chunks", input, split_sizes, sorted_idxs,
                              probs=probs, impl=impl)

    def __getattr__(self, name: str):
        if name.startswith("_"):
            raise AttributeError(name)
        if not self.registry.list(lambda s: s.op_name == name):
            raise AttributeError(name)

        def facade(*args: Any, impl: str | None = None, **kwargs: Any):
            return self._dispatch(name, *args, impl=impl, **kwargs)

        return facade


__all__ = ["OpDispatcher"]
