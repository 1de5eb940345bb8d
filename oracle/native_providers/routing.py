"""Native top-k routing (CPU oracle).

Restates ``topk_softmax_with_capacity`` and ``group_limited_topk`` of
``src/torchturbo/models/modules/moe/utils.py:30-80,127-230``:

* ``softmax``, post-top-k (default; Qwen3 ``norm_topk_prob`` and Mixtral):
  ``probs = softmax(topk(logits).values)`` in fp32 (``:190-196``);
* ``softmax``, pre-top-k: ``softmax(logits)`` in fp32, top-k of it (or of it
  plus the fp32 expert bias, then gathered) (``:181-189``);
* ``sigmoid`` / ``sqrtsoftplus``: fp32 scores, optional bias for selection
  only, renormalised with ``+1e-20`` when ``topk > 1`` (``:197-217``);
* group-limited selection: group score = sum of the top ``topk // group_topk``
  scores of each group; keep ``group_topk`` groups; top-k inside them (``:30-80``);
* token-id hash routing takes the ids from ``hash_table[input_ids]``;
* ``scaling_factor`` multiplies after normalisation (``:221-222``); probs are
  cast to the logits dtype (``:224``) and scattered to a dense [T, E] tensor
  and a boolean map (``:227-228``).

Ties: PyTorch's CPU ``topk`` has no documented tie rule. The HIP router
breaks ties toward the lower expert id; inputs used for bit-exact routing
comparisons use fp32 logits, where ties have measure zero (low-precision
comparisons skip rows whose k-th and (k+1)-th scores are equal), and the HIP
tie rule has its own test (``tests/test_gpu_ops.py``,
``test_router_ties_go_to_lower_expert``).

Pinned by: the KATs of ``tests/models/test_moe_router.py:74-171`` and
``tests/models/test_moe_adapter_routing.py:179-243`` restated in
``tests/test_oracle_kats.py`` and a brute-force sort on tiny inputs.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from torchturbo_amd.dispatch import OpImpl, OpImplKind, register_op


def group_limited_topk(scores, topk, num_tokens, num_experts, num_groups, group_topk):
    per_group = num_experts // num_groups
    group_scores = (
        scores.view(num_tokens, num_groups, per_group)
        .topk(topk // group_topk, dim=-1)[0].sum(dim=-1)
    )
    keep = torch.topk(group_scores, k=group_topk, dim=-1, sorted=False)[1]
    group_mask = torch.zeros_like(group_scores).scatter_(1, keep, 1)
    expert_mask = (
        group_mask.unsqueeze(-1).expand(num_tokens, num_groups, per_group)
        .reshape(num_tokens, num_experts)
    )
    masked = scores.masked_fill(~expert_mask.bool(), float("-inf"))
    return torch.topk(masked, k=topk, dim=-1)


def topk_softmax_with_capacity(
    logits, topk, use_pre_softmax=False, num_groups=None, group_topk=None,
    scaling_factor=None, score_function="softmax", expert_bias=None,
    use_hash_routing=False, hash_table=None, input_ids=None,
):
    assert logits.dim() == 2, f"Expected 2D logits [num_tokens, num_experts], got {logits.dim()}."
    num_tokens, num_experts = logits.shape

    def select(scores):
        if group_topk:
            return group_limited_topk(scores, topk, num_tokens, num_experts,
                                      num_groups, group_topk)
        return torch.topk(scores, k=topk, dim=1)

    if score_function == "softmax":
        if use_hash_routing:
            assert hash_table is not None and input_ids is not None
            top_indices = hash_table[input_ids]
        if use_pre_softmax:
            scores = torch.softmax(logits, dim=-1, dtype=torch.float32)
            if use_hash_routing:
                probs = scores.gather(1, top_indices)
            elif expert_bias is not None:
                top_indices = select(scores + expert_bias.float())[1]
                probs = scores.gather(1, top_indices)
            else:
                probs, top_indices = select(scores)
        else:
            if use_hash_routing:
                top_scores = logits.gather(1, top_indices)
            else:
                top_scores, top_indices = select(logits)
            probs = torch.softmax(top_scores, dim=-1, dtype=torch.float32)
    elif score_function in ("sigmoid", "sqrtsoftplus"):
        if score_function == "sigmoid":
            scores = torch.sigmoid(logits.float())
        else:
            scores = F.softplus(logits.float()).sqrt()
        if use_hash_routing:
            assert hash_table is not None and input_ids is not None
            top_indices = hash_table[input_ids]
            scores = scores.gather(1, top_indices)
        elif expert_bias is not None:
            top_indices = select(scores + expert_bias.float())[1]
            scores = scores.gather(1, top_indices)
        else:
            scores, top_indices = select(scores)
        probs = scores / (scores.sum(dim=-1, keepdim=True) + 1e-20) if topk > 1 else scores
    else:
        raise ValueError(f"Invalid score_function: {score_function}")

    if scaling_factor:
        probs = probs * scaling_factor
    probs = probs.type_as(logits)
    dense = torch.zeros_like(logits).scatter(1, top_indices, probs)
    routing_map = torch.zeros_like(logits).int().scatter(1, top_indices, 1).bool()
    return dense, routing_map, top_indices


@register_op(op_name="topk_softmax_with_capacity", impl_name="torch_topk_softmax",
             kind=OpImplKind.NATIVE, priority=0, devices=())
class TorchTopKSoftmax(OpImpl):
    def __call__(self, logits, topk, **kwargs):
        return topk_softmax_with_capacity(logits, topk, **kwargs)


def router_loss_stats(logits, topk, score_function="softmax", padding_mask=None, *,
                      aux=True, z=True):
    """The [T, E] sums behind the router's aux loss and z-loss.

    ``prob_sum`` / ``tokens_per_expert`` are ``scores.sum(0)`` and
    ``routing_map.sum(0)`` of ``compute_routing_scores_for_aux_loss``
    (``models/modules/moe/moe_utils.py:15-43``, bias-free scores, padding rows
    zeroed); ``z_sum`` is the fp32 sum of the valid rows of
    ``square(logsumexp(logits))`` (``moe_utils.py:61-68``), each value in the
    logits dtype. Switched-off parts are zeros.

    Pinned by: the aux/z KATs of ``tests/models/test_moe_router.py`` restated in
    ``tests/test_oracle_kats.py`` and closed forms on tiny inputs there.
    """
    logits = logits.reshape(-1, logits.size(-1))
    num_experts = logits.shape[1]
    prob_sum = torch.zeros(num_experts, dtype=torch.float32, device=logits.device)
    counts = torch.zeros(num_experts, dtype=torch.int64, device=logits.device)
    z_sum = torch.zeros((), dtype=torch.float32, device=logits.device)
    valid = None if padding_mask is None else (~padding_mask.reshape(-1).bool()).unsqueeze(-1)
    if aux:
        if score_function == "softmax":
            scores = torch.softmax(logits, dim=-1, dtype=torch.float32)
        elif score_function in ("sigmoid", "sqrtsoftplus"):
            scores = (torch.sigmoid(logits.float()) if score_function == "sigmoid"
                      else F.softplus(logits.float()).sqrt())
            scores = scores / (scores.sum(dim=-1, keepdim=True) + 1e-20)
        else:
            raise ValueError(f"Invalid score_function: {score_function}")
        top = torch.topk(scores, k=topk, dim=-1).indices
        routing_map = torch.zeros_like(logits, dtype=torch.int32).scatter_(1, top, 1).bool()
        if valid is not None:
            scores = scores * valid
            routing_map = (routing_map * valid).bool()
        prob_sum = scores.sum(dim=0)
        counts = routing_map.sum(dim=0)
    if z:
        values = torch.square(torch.logsumexp(logits, dim=-1))
        if valid is not None:
            values = values * valid.squeeze(-1)
        z_sum = values.float().sum()
    return prob_sum, counts, z_sum


@register_op(op_name="router_loss_stats", impl_name="torch_router_loss_stats",
             kind=OpImplKind.NATIVE, priority=0, devices=())
class TorchRouterLossStats(OpImpl):
    def __call__(self, logits, topk, score_function="softmax", padding_mask=None, *, aux=True,
                 z=True):
        return router_loss_stats(logits, topk, score_function, padding_mask, aux=aux, z=z)


def router_gate_topk(x, weight, router_dtype, topk, **kwargs):
    """``TopKRouter.gating`` (``router.py:25-58,84-101``: ``linear`` of the
    inputs and the weight cast to the router dtype, autocast off) followed by
    ``topk_softmax_with_capacity``; returns ``(probs, routing_map,
    top_indices, logits)``."""
    with torch.autocast(device_type=x.device.type, enabled=False):
        logits = F.linear(x.to(router_dtype), weight.to(router_dtype))
    logits2 = logits.reshape(-1, logits.shape[-1])
    if kwargs.get("input_ids") is not None:
        kwargs = {**kwargs, "input_ids": kwargs["input_ids"].reshape(-1)}
    probs, routing_map, top = topk_softmax_with_capacity(logits2, topk, **kwargs)
    return probs, routing_map, top, logits2


@register_op(op_name="router_gate_topk", impl_name="torch_router_gate_topk",
             kind=OpImplKind.NATIVE, priority=0, devices=())
class TorchRouterGateTopK(OpImpl):
    def __call__(self, x, weight, router_dtype, topk, **kwargs):
        return router_gate_topk(x, weight, router_dtype, topk, **kwargs)
