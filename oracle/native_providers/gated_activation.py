"""Native clamped gated activation (CPU oracle).

Restates ``src/torchturbo/ops/providers/native/gated_activation.py:15-44``:
``act(gate) * up`` on ``x = [gate, up]``; with ``limit > 0`` the math is in
fp32, ``up`` is clamped to ``[-limit, limit]`` and the gate is capped before
(``act(min(gate, limit))``) or after (``min(act(gate), limit)``) activation.
Only ``F.silu`` and ``F.gelu`` are accepted.

``gated_activation_probs`` is the composition
``GroupedMLP.activation_func_with_probs``
(``src/torchturbo/models/modules/moe/experts.py:181-186``):
``(gated_activation(x) * probs[:, None]).to(act.dtype)``.

Pinned by: closed form on hand-picked values (clamped / unclamped branches),
and gradcheck of the fp64 form away from the cap boundaries.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from torchturbo_amd.dispatch import OpImpl, OpImplKind, register_op

SUPPORTED = (F.silu, F.gelu)


def gated_activation(x, *, activation_func, limit: float = 0.0,
                     clamp_gate_after_activation: bool = False):
    if activation_func not in SUPPORTED:
        raise ValueError("gated_activation only supports F.silu and F.gelu.")
    limit = float(limit)
    if limit < 0:
        raise ValueError("limit must be non-negative.")
    gate, up = torch.chunk(x, 2, dim=-1)
    if limit == 0:
        return (activation_func(gate) * up).to(x.dtype)
    up = up.float().clamp(-limit, limit)
    if clamp_gate_after_activation:
        g = activation_func(gate.float()).clamp(max=limit)
    else:
        g = activation_func(gate.float().clamp(max=limit))
    return (g * up).to(x.dtype)


@register_op(op_name="gated_activation", impl_name="torch_gated_activation",
             kind=OpImplKind.NATIVE, priority=0, devices=())
class TorchGatedActivation(OpImpl):
    def __call__(self, x, *, activation_func, limit: float = 0.0,
                 clamp_gate_after_activation: bool = False):
        return gated_activation(x, activation_func=activation_func, limit=limit,
                                clamp_gate_after_activation=clamp_gate_after_activation)


def gated_activation_probs(x, probs, *, activation_func, limit: float = 0.0,
                           clamp_gate_after_activation: bool = False):
    act = gated_activation(x, activation_func=activation_func, limit=limit,
                           clamp_gate_after_activation=clamp_gate_after_activation)
    return (act * probs.unsqueeze(-1)).to(act.dtype)


@register_op(op_name="gated_activation_probs", impl_name="torch_gated_activation_probs",
             kind=OpImplKind.NATIVE, priority=0, devices=())
class TorchGatedActivationProbs(OpImpl):
    def __call__(self, x, probs, *, activation_func, limit: float = 0.0,
                 clamp_gate_after_activation: bool = False):
        return gated_activation_probs(x, probs, activation_func=activation_func, limit=limit,
                                      clamp_gate_after_activation=clamp_gate_after_activation)
