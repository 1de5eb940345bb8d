"""Token dispatcher for one GPU holding every expert (EP=1).

Keeps the six stages of ``MoEAlltoAllTokenDispatcher``
(``src/torchturbo/models/modules/moe/token_dispatcher.py:80-259``) and their
return values. With one expert-parallel rank:

* the token/prob exchange and the combine are the identity
  (``comm.py:147-150``), so ``token_dispatch``/``token_combine`` return their
  inputs;
* the local-expert chunk order is the identity (``token_dispatcher.py:101-107``),
  so no ``moe_sort_chunks`` call is made;
* per-expert counts stay on the device: the HIP grouped GEMM reads them there,
  so the reference's device->host copy and the wait at ``before_finish``
  (``:238-259``, ``experts.py:220-221``) are not needed.

Expert parallelism across GPUs is not part of this build; a dispatcher
constructed for more than one rank raises ``NotImplementedError``.
"""

from __future__ import annotations

import torch

from ..dispatch import MoEPermutation, ops
from .moe_config import MoEConfig


class MoETokenDispatcher:
    def __init__(self, config: MoEConfig, ep_group) -> None:
        self.config = config
        self.ep_size = config.expert_model_parallel_size or 1
        self.ep_group = ep_group


class MoEAlltoAllTokenDispatcher(MoETokenDispatcher):
    def __init__(self, num_local_experts: int, local_expert_indices: list[int],
                 config: MoEConfig, ep_group) -> None:
        super().__init__(config=config, ep_group=ep_group)
        if self.ep_size != 1:
            raise NotImplementedError(
                "This build runs the MoE expert path on one GPU holding every expert (EP=1)."
            )
        assert config.num_moe_experts is not None
        self.num_experts = config.num_moe_experts
        self.num_local_experts = num_local_experts
        assert num_local_experts == self.num_experts
        assert list(local_expert_indices) == list(range(num_local_experts))
        self.local_expert_indices = local_expert_indices
        self.hidden_shape = None
        self.hidden_shape_before_permute = None
        self.permutation_row_indices = None
        self.permutation_expert_indices = None
        self.tokens_per_expert = None

    def preprocess(self, routing_map: torch.Tensor) -> torch.Tensor:
        """Per-expert counts [E] int64, kept on the routing map's device."""
        return routing_map.sum(dim=0).long()

    def dispatch_preprocess(self, hidden_states, routing_map, probs, *, expert_indices=None):
        self.hidden_shape = hidden_states.shape
        assert probs.dim() == 2, "Expected 2D tensor for probs"
        assert routing_map.dim() == 2, "Expected 2D tensor for token2expert mask"
        assert routing_map.dtype == torch.bool, "Expected bool tensor for mask"
        hidden_states = hidden_states.view(-1, self.hidden_shape[-1])
        self.hidden_shape_before_permute = hidden_states.shape
        permutation = ops.moe_permutation(
            hidden_states, routing_map, probs=probs,
            num_out_tokens=routing_map.size(0) * self.config.moe_router_topk,
            expert_indices=expert_indices,
        )
        counts = getattr(permutation, "tokens_per_expert", None)
        self.tokens_per_expert = counts if counts is not None else self.preprocess(routing_map)
        self.permutation_row_indices = permutation.row_indices
        self.permutation_expert_indices = permutation.expert_indices
        return permutation.tokens, permutation.probs

    def token_dispatch(self, hidden_states, probs):
        return hidden_states, probs

    def dispatch_postprocess(self, hidden_states, probs):
        return hidden_states, self.tokens_per_expert, probs

    def combine_preprocess(self, hidden_states):
        return hidden_states

    def token_combine(self, hidden_states):
        return hidden_states

    def combine_postprocess(self, hidden_states):
        permutation = MoEPermutation(hidden_states, None, self.permutation_row_indices,
                                     self.permutation_expert_indices)
        output = ops.moe_unpermutation(permutation, restore_shape=self.hidden_shape_before_permute)
        output = output.view(self.hidden_shape)
        self.permutation_row_indices = None
        self.permutation_expert_indices = None
        return output
