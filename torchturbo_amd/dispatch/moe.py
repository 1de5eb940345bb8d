"""Shared tensor contract between ``moe_permutation`` and ``moe_unpermutation``.

Same fields and meaning as the reference's ``src/torchturbo/ops/moe.py:10-46``:
packed rows are expert-major, then ascending source token; every assignment
appears exactly once; ``row_indices[i, j]`` (int32) stays paired with
``expert_indices[i, j]`` (int64); slot order is free.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class MoEPermutation:
    # [num_tokens * topk, hidden] packed rows, source dtype, unweighted.
    tokens: torch.Tensor
    # [num_tokens * topk] routing weights in packed order (probs dtype), or None.
    probs: torch.Tensor | None
    # [num_tokens, topk] int32: packed row of each (token, slot).
    row_indices: torch.Tensor
    # [num_tokens, topk] int64: expert of each (token, slot).
    expert_indices: torch.Tensor


def get_expert_indices(routing_map: torch.Tensor) -> torch.Tensor:
    """Expert ids [T, k] from a boolean map with a uniform per-token count.

    Follows ``src/torchturbo/ops/moe.py:49-66``: ascending expert ids per
    token; ``ValueError`` when tokens select different numbers of experts.
    """
    num_tokens = routing_map.shape[0]
    if num_tokens == 0:
        return routing_map.new_empty((0, 0), dtype=torch.long)
    rows, experts = routing_map.nonzero(as_tuple=True)
    topk = experts.numel() // num_tokens
    expected_rows = (
        torch.arange(num_tokens, device=routing_map.device)
        .unsqueeze(1).expand(num_tokens, topk).reshape(-1)
    )
    if rows.numel() != expected_rows.numel() or not torch.equal(rows, expected_rows):
        raise ValueError("MoE permutation requires the same top-k count for every token.")
    return experts.view(num_tokens, topk)


__all__ = ["MoEPermutation", "get_expert_indices"]
