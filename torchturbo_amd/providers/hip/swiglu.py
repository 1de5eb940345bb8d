"""HIP SwiGLU providers.

``swiglu`` matches ``src/torchturbo/ops/providers/native/swiglu.py:10-24``;
``swiglu_probs`` fuses it with the expert probability weighting of
``GroupedMLP.activation_func_with_probs``
(``src/torchturbo/models/modules/moe/experts.py:181-186``) into one pass.
"""

from __future__ import annotations

from ...dispatch import OpImpl, OpImplKind, register_op
from ...runtime import TurboDevice
from . import PRIORITY
from ._functions import SwiGLU, require_cuda
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
