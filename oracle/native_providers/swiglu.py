"""Native SwiGLU and the expert probability weighting (CPU oracle).

* ``swiglu`` restates ``src/torchturbo/ops/providers/native/swiglu.py:10-12``:
  ``gate, up = chunk(x, 2)``; ``silu(gate)`` is rounded to ``x.dtype``, the
  product with ``up`` is rounded again.
* ``swiglu_probs`` is the composition ``GroupedMLP.activation_func_with_probs``
  (``src/torchturbo/models/modules/moe/experts.py:181-186``):
  ``(swiglu(x) * probs[:, None]).to(x.dtype)`` — the product is formed in the
  promoted dtype (fp32 when the router probabilities are fp32).

Pinned by: closed form on values where silu is exact at the rounding
points (``silu(0) = 0``), finite differences of the fp64 form, and the
bit-exact bf16 dense-loop KAT of
``tests/models/test_moe_probability_weighting.py:190-213``.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from torchturbo_amd.dispatch import OpImpl, OpImplKind, register_op


def swiglu(x: torch.Tensor) -> torch.Tensor:
    gate, up = torch.chunk(x, 2, dim=-1)
    return (F.silu(gate) * up).to(x.dtype)


def swiglu_probs(x: torch.Tensor, probs: torch.Tensor) -> torch.Tensor:
    act = swiglu(x)
    return (act * probs.unsqueeze(-1)).to(act.dtype)


@register_op(op_name="swiglu", impl_name="torch_swiglu",
             kind=OpImplKind.NATIVE, priority=0, devices=())
class TorchSwiGLU(OpImpl):
    def __call__(self, x):
        return swiglu(x)


@register_op(op_name="swiglu_probs", impl_name="torch_swiglu_probs",
             kind=OpImplKind.NATIVE, priority=0, devices=())
class TorchSwiGLUProbs(OpImpl):
    def __call__(self, x, probs):
        return swiglu_probs(x, probs)
