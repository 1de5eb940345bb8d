"""Operator dispatcher with the reference's selection policy and MoE facades.

Selection semantics follow ``src/torchturbo/ops/dispatcher.py:108-293``:

* construction resolves every registered op for the runtime's device and
  records (does not raise on) unresolved ones; an invalid config override
  raises ``RuntimeError`` at construction;
* an explicit ``impl=`` or an override never falls back (``148-160``);
* ``native`` / ``custom`` policies filter by kind and never cross over;
  ``auto`` walks the ranked candidates past unavailable ones (``162-186``);
* the first available candidate per (op, explicit impl) is remembered (a
  dispatcher serves one device).

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
from typing import Any

import torch

from ..runtime import DeviceRuntime
from .base import OpImpl, OpImplKind, OpPolicy, OpSpec
from .moe import MoEPermutation, get_expert_indices
from .providers import iter_provider_modules
from .registry import OpRegistry

logger = logging.getLogger("torchturbo_amd")


def _impl_classes_of(module_names) -> dict[str, type[OpImpl]]:
    """impl_name -> ``OpImpl`` subclass, over the classes that the given
    provider modules define themselves (not import) and that carry an
    ``OpSpec``. One impl_name bound to two different classes is an error."""
    found: dict[str, list[type[OpImpl]]] = {}
    for module_name in module_names:
        module = importlib.import_module(module_name)
        for obj in vars(module).values():
            if (isinstance(obj, type) and obj is not OpImpl and issubclass(obj, OpImpl)
                    and obj.__module__ == module.__name__
                    and getattr(obj, "__op_spec__", None) is not None):
                bucket = found.setdefault(obj.__op_spec__.impl_name, [])
                if obj not in bucket:
                    bucket.append(obj)
    for impl_name, bucket in found.items():
        if len(bucket) > 1:
            first, second = bucket[0], bucket[1]
            raise ValueError(
                f"Op implementation {impl_name!r} is defined by both "
                f"{first.__module__}.{first.__qualname__} and "
                f"{second.__module__}.{second.__qualname__}."
            )
    return {impl_name: bucket[0] for impl_name, bucket in found.items()}


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
        self._device = device_runtime.turbo_device
        self._impl_classes = _impl_classes_of(iter_provider_modules(self._device))
        self._instances: dict[str, OpImpl] = {}
        # (op, explicit impl or None) -> (chosen spec, whether ranked candidates
        # before it were unavailable)
        self._chosen: dict[tuple[str, str | None], tuple[OpSpec, bool]] = {}
        self._unresolved_ops: dict[str, str] = {}
        self._resolve_all()

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

    # -- resolution --------------------------------------------------------
    def _resolve_all(self) -> None:
        """Resolve every op the device has providers for. Overrides are checked
        first and a bad one raises; an op with no usable implementation is only
        recorded (it raises when called)."""
        here = self.registry.list(lambda s: not s.devices or self._device in s.devices)
        provided = {s.op_name for s in here if s.impl_name in self._impl_classes}
        for op_name, impl_name in sorted(self._overrides.items()):
            try:
                self._resolve(op_name, impl_name)
            except RuntimeError as exc:
                raise RuntimeError(
                    f"Invalid override for op {op_name!r}: {impl_name!r}. {exc}"
                ) from exc
        for op_name in sorted(provided - set(self._overrides)):
            try:
                self._resolve(op_name, None)
            except RuntimeError as exc:
                self._unresolved_ops[op_name] = str(exc)

    def _policy_admits(self, spec: OpSpec) -> bool:
        if self._default_policy == OpPolicy.NATIVE:
            return spec.kind == OpImplKind.NATIVE
        if self._default_policy == OpPolicy.CUSTOM:
            return spec.kind == OpImplKind.CUSTOM
        return True

    def _ranked(self, op_name: str, impl: str | None) -> list[OpSpec]:
        """The specs to try for ``op_name``: the named one only (no fallback), or
        the policy's candidates for this device, best first."""
        device = self._device
        if impl is None:
            return self.registry.list(
                lambda s: (s.op_name == op_name and s.impl_name in self._impl_classes
                           and (not s.devices or device in s.devices)
                           and self._policy_admits(s)))
        spec = self.registry.get_by_impl_name(impl)
        if spec.op_name != op_name:
            raise RuntimeError(
                f"Implementation {impl!r} is registered for op {spec.op_name!r}, not {op_name!r}."
            )
        if spec.devices and device not in spec.devices:
            raise RuntimeError(
                f"Implementation {impl!r} for op {op_name!r} does not support "
                f"device={device.value}."
            )
        return [spec]

    def _instance(self, spec: OpSpec) -> OpImpl:
        try:
            return self._instances[spec.impl_name]
        except KeyError:
            pass
        cls = self._impl_classes.get(spec.impl_name)
        if cls is None:
            raise RuntimeError(f"No OpImpl class registered for impl_name {spec.impl_name!r}.")
        return self._instances.setdefault(spec.impl_name, cls())

    def _resolve(self, op_name: str, impl: str | None) -> OpImpl:
        """The implementation ``op_name`` runs (first available candidate,
        remembered per (op, explicit impl))."""
        hit = self._chosen.get((op_name, impl))
        if hit is not None:
            return self._instances[hit[0].impl_name]
        skipped = []
        for spec in self._ranked(op_name, impl):
            obj = self._instance(spec)
            if obj.available():
                self._chosen[(op_name, impl)] = (spec, bool(skipped))
                return obj
            skipped.append(spec.impl_name)
        how = f"policy={self._default_policy.value}" if impl is None else f"impl={impl}"
        why = f" (unavailable={skipped})" if skipped else ""
        raise RuntimeError(
            f"No implementation for op={op_name!r}, device={self._device.value}, {how}{why}."
        )

    def selected_impl_name(self, op_name: str) -> str:
        """Name of the implementation the dispatcher would run for ``op_name``."""
        override = self._overrides.get(op_name)
        self._resolve(op_name, override)
        return self._chosen[(op_name, override)][0].impl_name

    def log_ops_selection(self) -> str:
        """Log (and return) the op → implementation table (``dispatcher.py:213-277``)."""
        rows = []
        chosen = {op: hit for (op, impl), hit in self._chosen.items()
                  if impl == self._overrides.get(op)}
        for op_name in sorted(set(chosen) | set(self._unresolved_ops)):
            hit = chosen.get(op_name)
            if hit is None:
                rows.append((op_name, "-", "-", "-", "unavailable"))
                continue
            spec, fell_back = hit
            status = ("overridden" if op_name in self._overrides
                      else "fallback" if fell_back else "selected")
            rows.append((op_name, spec.impl_name, spec.kind.value, str(spec.priority), status))
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
        selected = impl if impl is not None else self._overrides.get(op_name)
        return self._resolve(op_name, selected)(*args, **kwargs)

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
