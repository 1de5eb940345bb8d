"""Native mask permutation, unpermutation and chunk sort (CPU oracle).

Restates ``src/torchturbo/ops/providers/native/moe_permutation.py``:

* permutation (``:25-57``): packed order = experts ascending, tokens
  ascending within an expert; ``row_indices[t, j]`` is the packed row of the
  assignment ``(t, expert_indices[t, j])``; probs are gathered in packed
  order keeping their dtype;
* unpermutation (``:68-99``): optional weighting by
  ``probs[t, expert_indices[t, j]]`` in the probs dtype, then the rows of a
  token are accumulated in ascending packed-row order — PyTorch's CPU
  ``scatter_add_``/``index_add_`` on bf16/fp16 accumulate in fp32 and round
  once (probed on torch 2.10; pinned by the KAT of
  ``tests/ops/test_moe_permutation_contract.py:37-69``);
* chunk sort (``:110-126``): host split + concatenation in ``sorted_idxs``
  order.

Pinned by: brute-force pair sorting (``oracle/route_np.py``) and the literal
KATs of ``tests/ops/test_moe_permutation_contract.py:72-84,307-370,412-434``
(see ``tests/test_oracle_kats.py``).
"""

from __future__ import annotations

import torch

from torchturbo_amd.dispatch import MoEPermutation, OpImpl, OpImplKind, register_op


def packed_order(routing_map: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(source token of each packed row, packed row of each [T, E] cell)."""
    num_tokens, num_experts = routing_map.shape
    expert_major = routing_map.bool().t().contiguous()  # [E, T]
    flat = expert_major.reshape(-1)
    cell = torch.nonzero(flat, as_tuple=False).reshape(-1)  # ascending (e, t)
    token_of_row = cell % max(num_tokens, 1)
    row_of_cell = torch.full((num_experts * num_tokens,), -1, dtype=torch.int32)
    row_of_cell[cell] = torch.arange(cell.numel(), dtype=torch.int32)
    return token_of_row, row_of_cell.view(num_experts, num_tokens).t()


def permute(tokens, routing_map, probs=None, expert_indices=None) -> MoEPermutation:
    token_of_row, row_of_cell = packed_order(routing_map)
    packed = tokens.index_select(0, token_of_row)
    packed_probs = None
    if probs is not None:
        # Same (expert, token) cell order as the token rows; autograd flows
        # back to the dense ``probs``.
        packed_probs = probs.t()[routing_map.bool().t()]
    if expert_indices is None:
        raise ValueError("expert_indices is required")
    rows = row_of_cell.gather(1, expert_indices) if expert_indices.numel() else \
        torch.empty(expert_indices.shape, dtype=torch.int32)
    return MoEPermutation(packed, packed_probs, rows.to(torch.int32), expert_indices)


def unpermute(permutation: MoEPermutation, restore_shape, probs=None) -> torch.Tensor:
    values = permutation.tokens
    out_dtype = values.dtype
    num_tokens, topk = permutation.row_indices.shape
    rows = permutation.row_indices.reshape(-1).long()
    source = torch.arange(num_tokens).unsqueeze(1).expand(num_tokens, topk).reshape(-1)
    token_of_row = torch.empty_like(source)
    token_of_row[rows] = source
    if probs is not None:
        chosen = probs.gather(1, permutation.expert_indices).reshape(-1)
        weight_of_row = torch.empty_like(chosen).scatter(0, rows, chosen)
        values = values * weight_of_row.unsqueeze(-1)
    out = values.new_zeros(restore_shape)
    # Ascending packed rows, fp32 accumulation for reduced types, one rounding.
    out = out.index_add(0, token_of_row, values)
    return out.to(out_dtype)


def sort_chunks(input, split_sizes, sorted_idxs, probs=None):
    sizes = [int(s) for s in split_sizes.cpu().tolist()]
    order = [int(i) for i in sorted_idxs.cpu().tolist()]
    parts = torch.split(input, sizes, dim=0)
    out = torch.cat([parts[i] for i in order], dim=0)
    out_probs = None
    if probs is not None:
        pparts = torch.split(probs, sizes, dim=0)
        out_probs = torch.cat([pparts[i] for i in order], dim=0)
    return out, out_probs


@register_op(op_name="moe_permutation", impl_name="torch_moe_mask_permutation",
             kind=OpImplKind.NATIVE, priority=0, devices=())
class TorchMoEMaskPermutation(OpImpl):
    def __call__(self, tokens, routing_map, probs=None, num_out_tokens=None,
                 expert_indices=None) -> MoEPermutation:
        return permute(tokens, routing_map, probs=probs, expert_indices=expert_indices)


@register_op(op_name="moe_unpermutation", impl_name="torch_moe_mask_unpermutation",
             kind=OpImplKind.NATIVE, priority=0, devices=())
class TorchMoEMaskUnpermutation(OpImpl):
    def __call__(self, permutation, restore_shape, probs=None) -> torch.Tensor:
        return unpermute(permutation, restore_shape, probs=probs)


@register_op(op_name="moe_sort_chunks", impl_name="torch_moe_sort_chunks",
             kind=OpImplKind.NATIVE, priority=0, devices=())
class TorchMoESortChunks(OpImpl):
    def __call__(self, input, split_sizes, sorted_idxs, probs=None):
        return sort_chunks(input, split_sizes, sorted_idxs, probs=probs)
