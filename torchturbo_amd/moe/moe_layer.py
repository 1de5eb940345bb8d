"""MoE layer: router -> dispatcher -> experts -> combine.

Mirrors ``MoELayer`` (``src/torchturbo/models/modules/moe/moe_layer.py:94-183``):
same constructor, ``forward(hidden_states, input_ids=None) -> (output,
logits)`` and shared-expert handling. ``forward_with_logits`` runs the same
path from router logits supplied by the caller (the benchmark feeds synthetic
logits of a given distribution, as the reference's configurations state).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Union

import torch
import torch.distributed as dist
import torch.nn.functional as F

from ..dispatch import ops
from .experts import GroupedMLP
from .module import ModuleSpec, build_module
from .moe_config import MoEConfig
from .router import TopKRouter
from .token_dispatcher import MoEAlltoAllTokenDispatcher


@dataclass
class MoESubmodules:
    experts: Union[ModuleSpec, type] = None
    shared_experts: Union[ModuleSpec, type] = None


@dataclass
class MoERuntimeInputs:
    padding_mask: torch.Tensor | None = None
    accumulate_tokens_per_expert: bool = True


def _group_size_rank(group) -> tuple[int, int]:
    if group is None or not dist.is_available() or not dist.is_initialized():
        return 1, 0
    return dist.get_world_size(group), dist.get_rank(group)


class BaseMoELayer(torch.nn.Module):
    def __init__(self, config: MoEConfig, ep_group, layer_number: Optional[int] = None):
        super().__init__()
        ep_size, ep_rank = _group_size_rank(ep_group)
        self.config = config
        self.expert_parallel_size = ep_size
        assert config.num_moe_experts % ep_size == 0
        self.num_local_experts = config.num_moe_experts // ep_size
        offset = ep_rank * self.num_local_experts
        self.use_shared_expert = config.moe_shared_expert_intermediate_size is not None
        self.local_expert_indices = [offset + i for i in range(self.num_local_experts)]
        self.router = None
        self.experts = None
        self.shared_experts = None
        self.shared_expert = None
        self.shared_expert_gate = None
        self.token_dispatcher = None
        self.layer_number = layer_number
        self._runtime_inputs = MoERuntimeInputs()

    def set_runtime_inputs(self, inputs: MoERuntimeInputs) -> None:
        self._runtime_inputs = inputs


class MoELayer(BaseMoELayer):
    """Mixture-of-experts layer without token dropping."""

    def __init__(self, config: MoEConfig, ep_group=None, submodules: Optional[MoESubmodules] = None,
                 use_te: bool = False, layer_number: Optional[int] = None, sp_group=None):
        self.use_te = use_te
        self.submodules = submodules
        super().__init__(config=config, ep_group=ep_group, layer_number=layer_number)
        self.router = TopKRouter(config=config, layer_number=layer_number, sp_group=sp_group)
        if config.moe_token_dispatcher_type != "alltoall":
            raise ValueError(
                f"Unsupported token dispatcher type: {config.moe_token_dispatcher_type}")
        self.token_dispatcher = MoEAlltoAllTokenDispatcher(
            self.num_local_experts, self.local_expert_indices, config=config, ep_group=ep_group)
        self.experts = build_module(submodules.experts, self.num_local_experts, use_te, config,
                                    layer_number=layer_number)
        if self.use_shared_expert:
            self.shared_experts = build_module(submodules.shared_experts, config=config)

    def _gathering_experts(self, tokens, expert_indices) -> bool:
        """Whether the permutation and unpermutation can be folded into the
        experts' GEMMs (HIP providers for the three ops, plain ``GroupedMLP``
        experts; shapes in ``providers.hip.fused_experts.eligible``)."""
        if type(self.experts) is not GroupedMLP or self.config.moe_apply_probs_on_input:
            return False
        if expert_indices is None or not tokens.is_cuda:
            return False
        try:
            chosen = (ops.selected_impl_name("moe_permutation"),
                      ops.selected_impl_name("grouped_matmul"),
                      ops.selected_impl_name("moe_unpermutation"))
        except RuntimeError:
            return False
        if chosen != ("hip_moe_mask_permutation", "hip_grouped_matmul",
                      "hip_moe_mask_unpermutation"):
            return False
        from ..providers.hip import fused_experts
        return fused_experts.eligible(tokens, self.experts.weight1, expert_indices.shape[1],
                                      self.num_local_experts)

    def _experts_and_combine(self, hidden_states, probs, routing_map, expert_indices):
        flat = hidden_states.view(-1, hidden_states.shape[-1])
        if self._gathering_experts(flat, expert_indices):
            # One GPU, every expert local: the GEMMs gather the token rows
            # themselves (same results, no packed copies).
            from ..providers.hip import fused_experts
            tokens, counts = fused_experts.grouped_mlp_tokens(self.experts, flat, probs,
                                                              routing_map, expert_indices)
            self.token_dispatcher.tokens_per_expert = counts
            output = tokens.view(hidden_states.shape).to(hidden_states.dtype)
        else:
            output = self._dispatched_experts(hidden_states, probs, routing_map, expert_indices)
        if self.shared_expert is not None:
            shared = self.shared_expert(hidden_states)
            output = output + F.sigmoid(self.shared_expert_gate(hidden_states)) * shared
        if self.shared_experts is not None:
            output = output + self.shared_experts(hidden_states)
        return output

    def _dispatched_experts(self, hidden_states, probs, routing_map, expert_indices):
        d = self.token_dispatcher
        tokens, expert_probs = d.dispatch_preprocess(hidden_states, routing_map, probs,
                                                     expert_indices=expert_indices)
        tokens, expert_probs = d.token_dispatch(tokens, expert_probs)
        tokens, tokens_per_expert, expert_probs = d.dispatch_postprocess(tokens, expert_probs)
        tokens, bias = self.experts(tokens, tokens_per_expert, expert_probs)
        assert bias is None
        tokens = d.combine_preprocess(tokens)
        tokens = d.token_combine(tokens)
        tokens = d.combine_postprocess(tokens)
        return tokens.to(hidden_states.dtype)

    def forward(self, hidden_states, input_ids=None):
        probs, routing_map, expert_indices, logits = self.router(
            hidden_states, input_ids, self._runtime_inputs.padding_mask,
            self._runtime_inputs.accumulate_tokens_per_expert)
        logits = logits.view(-1, logits.shape[-1])
        return self._experts_and_combine(hidden_states, probs, routing_map, expert_indices), logits

    def forward_with_logits(self, hidden_states, logits, input_ids=None):
        """Same path with caller-supplied router logits [T, E]."""
        probs, routing_map, expert_indices = self.router.routing(
            logits, input_ids, self._runtime_inputs.padding_mask,
            self._runtime_inputs.accumulate_tokens_per_expert)
        return self._experts_and_combine(hidden_states, probs, routing_map, expert_indices)
