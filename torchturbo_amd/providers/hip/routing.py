"""HIP top-k router provider.

Implements ``topk_softmax_with_capacity``
(``src/torchturbo/models/modules/moe/utils.py:127-230``) in one kernel per
direction: score function, optional expert bias (selection only),
group-limited selection, top-k, normalisation, scaling, the cast to the
logits dtype and the dense probs / boolean map, with its autograd backward.
Ties between equal scores go to the lower expert id.
"""

from __future__ import annotations

from ...dispatch import OpImpl, OpImplKind, register_op
from ...runtime import TurboDevice
from . import PRIORITY
from ._functions import RouterGateTopK, RouterLossStats, TopKRouting, require_cuda
from .available import hip_available


@register_op(op_name="topk_softmax_with_capacity", impl_name="hip_topk_softmax",
             kind=OpImplKind.CUSTOM, priority=PRIORITY, devices=(TurboDevice.CUDA,))
class HipTopKSoftmax(OpImpl):
    def available(self) -> bool:
        return hip_available()

    def __call__(self, logits, topk, use_pre_softmax=False, num_groups=None, group_topk=None,
                 scaling_factor=None, score_function="softmax", expert_bias=None,
                 use_hash_routing=False, hash_table=None, input_ids=None):
        require_cuda(logits)
        if logits.dim() != 2:
            raise ValueError(f"Expected 2D logits [num_tokens, num_experts], got {logits.dim()}.")
        if score_function not in ("softmax", "sigmoid", "sqrtsoftplus"):
            raise ValueError(f"Invalid score_function: {score_function}")
        fixed = None
        if use_hash_routing:
            if hash_table is None or input_ids is None:
                raise ValueError("Hash routing requires hash_table and input_ids.")
            fixed = hash_table.to(logits.device)[input_ids.to(logits.device)]
        bias = expert_bias if score_function != "softmax" or use_pre_softmax else None
        return TopKRouting.apply(logits, int(topk), score_function, bool(use_pre_softmax),
                                 num_groups, group_topk, scaling_factor, bias, fixed)


@register_op(op_name="router_loss_stats", impl_name="hip_router_loss_stats",
             kind=OpImplKind.CUSTOM, priority=PRIORITY, devices=(TurboDevice.CUDA,))
class HipRouterLossStats(OpImpl):
    """``(prob_sum [E], tokens_per_expert [E], z_sum [])``: the [T, E] sums of
    the router's aux loss (``moe_utils.py:15-43``, ``router.py:164-209``) and
    z-loss (``moe_utils.py:46-70``, ``router.py:225-270``) in one kernel pass
    per direction, instead of the softmax / top-k / scatter / reductions of
    the native composition."""

    def available(self) -> bool:
        return hip_available()

    def __call__(self, logits, topk, score_function="softmax", padding_mask=None, *, aux=True,
                 z=True):
        require_cuda(logits)
        if logits.dim() != 2:
            raise ValueError(f"Expected 2D logits [num_tokens, num_experts], got {logits.dim()}.")
        if score_function not in ("softmax", "sigmoid", "sqrtsoftplus"):
            raise ValueError(f"Invalid score_function: {score_function}")
        if aux and not 1 <= int(topk) <= logits.shape[1]:
            raise ValueError(f"topk must be in [1, {logits.shape[1]}], got {topk}")
        return RouterLossStats.apply(logits, int(topk), score_function, padding_mask, bool(aux),
                                     bool(z))


@register_op(op_name="router_gate_topk", impl_name="hip_router_gate_topk",
             kind=OpImplKind.CUSTOM, priority=PRIORITY, devices=(TurboDevice.CUDA,))
class HipRouterGateTopK(OpImpl):
    """``(probs, routing_map, top_indices, logits)`` of ``TopKRouter.gating``
    (``router.py:25-58,84-101``) followed by ``topk_softmax_with_capacity``
    (``utils.py:127-230``), in one kernel: x and the router weight in bf16 or
    f16 (the same dtype), logits in that dtype or fp32, E a multiple of 32 up
    to 256, hidden a multiple of 64 (``TopKRouter`` checks this before it
    asks)."""

    def available(self) -> bool:
        return hip_available()

    def __call__(self, x, weight, router_dtype, topk, use_pre_softmax=False, num_groups=None,
                 group_topk=None, scaling_factor=None, score_function="softmax",
                 expert_bias=None, use_hash_routing=False, hash_table=None, input_ids=None):
        require_cuda(x, weight)
        if score_function not in ("softmax", "sigmoid", "sqrtsoftplus"):
            raise ValueError(f"Invalid score_function: {score_function}")
        fixed = None
        if use_hash_routing:
            if hash_table is None or input_ids is None:
                raise ValueError("Hash routing requires hash_table and input_ids.")
            fixed = hash_table.to(x.device)[input_ids.reshape(-1).to(x.device)]
        bias = expert_bias if score_function != "softmax" or use_pre_softmax else None
        return RouterGateTopK.apply(x, weight, router_dtype, int(topk), score_function,
                                    bool(use_pre_softmax), num_groups, group_topk,
                                    scaling_factor, bias, fixed)
