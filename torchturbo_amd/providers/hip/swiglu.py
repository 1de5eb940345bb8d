"""HIP SwiGLU providers.

``swiglu`` matches ``src/torchturbo/ops/providers/native/swiglu.py:10-24``;
``swiglu_probs`` fuses it with the expert probability weighting of
``GroupedMLP.activation_func_with_probs``
(``src/torchturbo/models/modules/moe/experts.py:181-186``) into one pass.
``gated_activation`` matches
``src/torchturbo/ops/providers/native/gated_activation.py:15-68`` (SiLU or GELU
gate, optional cap); ``gated_activation_probs`` fuses it with the probability
product the same way.
"""

from __future__ import annotations

from ...dispatch import OpImpl, OpImplKind, register_op
from ...runtime import TurboDevice
from . import PRIORITY
import torch.nn.functional as F

from ._functions import GatedActivation, SwiGLU, require_cuda
from .available import hip_available


def _flat2d(x):
    return x.reshape(-1, x.shape[-1])


@register_op(op_name="swiglu", impl_name="hip_swiglu",
             kind=OpImplKind.CUSTOM, priority=PRIORITY, devices=(TurboDevice.CUDA,))
class HipSwiGLU(OpImpl):
    def available(self) -> bool:
        return hip_available()

    def __call__(self, x):
        require_cuda(x)
        out = SwiGLU.apply(_flat2d(x), None)
        return out.view(*x.shape[:-1], x.shape[-1] // 2)


@register_op(op_name="swiglu_probs", impl_name="hip_swiglu_probs",
             kind=OpImplKind.CUSTOM, priority=PRIORITY, devices=(TurboDevice.CUDA,))
class HipSwiGLUProbs(OpImpl):
    def available(self) -> bool:
        return hip_available()

    def __call__(self, x, probs):
        require_cuda(x, probs)
        flat = _flat2d(x)
        p = probs.reshape(-1)
        if p.numel() != flat.shape[0]:
            raise ValueError("swiglu_probs expects one probability per row")
        out = SwiGLU.apply(flat, p)
        return out.view(*x.shape[:-1], x.shape[-1] // 2)


def _act_code(activation_func) -> int:
    if activation_func is F.silu:
        return 0
    if activation_func is F.gelu:
        return 1
    raise ValueError("gated_activation only supports F.silu and F.gelu.")


def _limit(limit) -> float:
    limit = float(limit)
    if limit < 0:
        raise ValueError("limit must be non-negative.")
    return limit


@register_op(op_name="gated_activation", impl_name="hip_gated_activation",
             kind=OpImplKind.CUSTOM, priority=PRIORITY, devices=(TurboDevice.CUDA,))
class HipGatedActivation(OpImpl):
    def available(self) -> bool:
        return hip_available()

    def __call__(self, x, *, activation_func, limit: float = 0.0,
                 clamp_gate_after_activation: bool = False):
        act, lim = _act_code(activation_func), _limit(limit)
        require_cuda(x)
        out = GatedActivation.apply(_flat2d(x), None, act, lim, clamp_gate_after_activation)
        return out.view(*x.shape[:-1], x.shape[-1] // 2)


@register_op(op_name="gated_activation_probs", impl_name="hip_gated_activation_probs",
             kind=OpImplKind.CUSTOM, priority=PRIORITY, devices=(TurboDevice.CUDA,))
class HipGatedActivationProbs(OpImpl):
    def available(self) -> bool:
        return hip_available()

    def __call__(self, x, probs, *, activation_func, limit: float = 0.0,
                 clamp_gate_after_activation: bool = False):
        act, lim = _act_code(activation_func), _limit(limit)
        require_cuda(x, probs)
        flat = _flat2d(x)
        p = probs.reshape(-1)
        if p.numel() != flat.shape[0]:
            raise ValueError("gated_activation_probs expects one probability per row")
        out = GatedActivation.apply(flat, p, act, lim, clamp_gate_after_activation)
        return out.view(*x.shape[:-1], x.shape[-1] // 2)
