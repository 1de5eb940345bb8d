"""HIP mask permutation, unpermutation and chunk sort.

Same facade contract as the reference providers
(``src/torchturbo/ops/providers/native/moe_permutation.py``,
``ops/providers/cuda/moe_permutation.py:38-197``): packed rows are
expert-major then token-ascending, ``row_indices`` int32 [T, k] paired with
``expert_indices`` int64 [T, k], probs gathered in packed order keeping their
dtype; unpermutation sums a token's rows (weighted by
``probs[t, expert_indices[t, j]]`` when probs are given) in fp32 and rounds
once. The returned ``MoEPermutation`` also carries the per-expert counts the
index build produced (``tokens_per_expert``, int64 on the device), so callers
need no separate reduction of the routing map.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ... import _lib as L
from ... import checks
from ...dispatch import MoEPermutation, OpImpl, OpImplKind, register_op
from ...runtime import TurboDevice
from . import PRIORITY
from ._functions import Permute, Unpermute, require_cuda
from .available import hip_available


@dataclass(frozen=True)
class HipMoEPermutation(MoEPermutation):
    tokens_per_expert: torch.Tensor | None = None


@register_op(op_name="moe_permutation", impl_name="hip_moe_mask_permutation",
             kind=OpImplKind.CUSTOM, priority=PRIORITY, devices=(TurboDevice.CUDA,))
class HipMoEMaskPermutation(OpImpl):
    def available(self) -> bool:
        return hip_available()

    def __call__(self, tokens, routing_map, probs=None, num_out_tokens=None,
                 expert_indices=None) -> MoEPermutation:
        require_cuda(tokens, routing_map, probs, expert_indices)
        if tokens.dim() != 2:
            raise ValueError("moe_permutation expects tokens of shape [num_tokens, hidden].")
        num_experts = routing_map.shape[1]
        if expert_indices is None:
            raise ValueError("expert_indices is required")
        if expert_indices.shape[0] != tokens.shape[0]:
            raise ValueError("expert_indices must have one row per token")
        if routing_map.shape[0] != tokens.shape[0]:
            raise ValueError("routing_map must have one row per token")
        packed, pprobs, rows, counts = Permute.apply(tokens, probs, expert_indices, num_experts)
        if checks.enabled():  # after the id check inside the routing index
            _check_map_matches_indices(routing_map, expert_indices)
        return HipMoEPermutation(packed, pprobs, rows, expert_indices, counts)


def _check_map_matches_indices(routing_map, expert_indices):
    """The packed order comes from expert_indices alone; the reference builds it
    from routing_map (native/moe_permutation.py:36-51) and requires the two to
    agree (ops/dispatcher.py:559-562). Ids outside [0, E) and repeated ids are
    caught by the routing index itself."""
    T, K = expert_indices.shape
    if T == 0:
        return
    per_token = routing_map.bool().sum(dim=1)
    ids = expert_indices.clamp(0, routing_map.shape[1] - 1)
    agree = routing_map.bool().gather(1, ids).all(dim=1) & (per_token == K)
    if not bool(agree.all()):
        bad = int((~agree).sum())
        raise ValueError(
            f"routing_map and expert_indices disagree for {bad} of {T} tokens: each token's "
            f"routing_map row must select exactly its {K} expert_indices."
        )


@register_op(op_name="moe_unpermutation", impl_name="hip_moe_mask_unpermutation",
             kind=OpImplKind.CUSTOM, priority=PRIORITY, devices=(TurboDevice.CUDA,))
class HipMoEMaskUnpermutation(OpImpl):
    def available(self) -> bool:
        return hip_available()

    def __call__(self, permutation: MoEPermutation, restore_shape, probs=None) -> torch.Tensor:
        require_cuda(permutation.tokens, permutation.row_indices, probs)
        num_tokens = int(restore_shape[0])
        if permutation.row_indices.shape[0] != num_tokens:
            raise ValueError("restore_shape must match the token count of row_indices")
        if permutation.tokens.shape[-1] != int(restore_shape[-1]):
            raise ValueError("restore_shape must match the feature width of the packed tokens")
        out = Unpermute.apply(permutation.tokens, permutation.row_indices,
                              permutation.expert_indices, probs, num_tokens)
        return out.view(restore_shape)


@register_op(op_name="moe_sort_chunks", impl_name="hip_moe_sort_chunks",
             kind=OpImplKind.CUSTOM, priority=PRIORITY, devices=(TurboDevice.CUDA,))
class HipMoESortChunks(OpImpl):
    """Chunk reorder on the device (metadata never leaves the GPU)."""

    def available(self) -> bool:
        return hip_available()

    def __call__(self, input, split_sizes, sorted_idxs, probs=None):
        require_cuda(input, split_sizes, sorted_idxs, probs)
        if split_sizes.dim() != 1 or sorted_idxs.dim() != 1:
            raise ValueError("moe_sort_chunks expects 1-D split_sizes and sorted_idxs.")
        if split_sizes.numel() != sorted_idxs.numel():
            raise ValueError(
                f"moe_sort_chunks: {sorted_idxs.numel()} chunk ids for "
                f"{split_sizes.numel()} chunks; sorted_idxs must order every chunk once."
            )
        if probs is not None and probs.shape[0] != input.shape[0]:
            raise ValueError("moe_sort_chunks: probs must have one entry per input row.")
        if checks.enabled():
            _check_chunks(input.shape[0], split_sizes, sorted_idxs)
        return _SortChunks.apply(input, probs, split_sizes, sorted_idxs)


def _check_chunks(rows, sizes, order):
    """What torch.split / the chunk loop of the reference reject
    (native/moe_permutation.py:117-119): sizes that do not cover the rows
    exactly, negative sizes, or an order that is not a permutation."""
    C = sizes.numel()
    total = int(sizes.sum()) if C else 0
    if total != rows or (C and int(sizes.min()) < 0):
        raise ValueError(f"moe_sort_chunks: split_sizes sum to {total}, the input has {rows} rows.")
    seen = torch.zeros(C, dtype=torch.int64, device=order.device)
    valid = bool(((order >= 0) & (order < C)).all()) if C else True
    if valid and C:
        seen.index_add_(0, order.long(), torch.ones_like(order, dtype=torch.int64))
    if not valid or not bool((seen == 1).all()):
        raise ValueError("moe_sort_chunks: sorted_idxs must be a permutation of the chunk ids.")


def _sort_chunks(x, probs, sizes, order):
    x = x.contiguous()
    rows = x.shape[0]
    hidden = x[0].numel() if rows else (x.shape[1] if x.dim() > 1 else 1)
    out = torch.empty_like(x)
    out_p = torch.empty_like(probs) if probs is not None else None
    sizes = sizes.to(torch.int64).contiguous()
    order = order.to(torch.int64).contiguous()
    pc = probs.contiguous() if probs is not None else None
    L.call("tt_sort_chunks", L.ptr(x), L.dtype_code(x.dtype), rows, hidden, L.ptr(sizes),
           L.ptr(order), int(order.numel()), L.ptr(pc),
           L.dtype_code(probs.dtype) if probs is not None else 0, L.ptr(out), L.ptr(out_p),
           L.stream(x.device))
    return out, out_p


def _inverse_order(sizes, order):
    """Split sizes and order that undo a chunk reorder."""
    inv = torch.empty_like(order)
    inv[order] = torch.arange(order.numel(), device=order.device, dtype=order.dtype)
    return sizes[order], inv


class _SortChunks(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, probs, sizes, order):
        out, out_p = _sort_chunks(x, probs, sizes, order)
        ctx.save_for_backward(sizes, order)
        ctx.has_probs = probs is not None
        return out, out_p

    @staticmethod
    def backward(ctx, g_out, g_probs):
        sizes, order = ctx.saved_tensors
        inv_sizes, inv_order = _inverse_order(sizes.to(torch.int64), order.to(torch.int64))
        gx, gp = _sort_chunks(g_out, g_probs if ctx.has_probs else None, inv_sizes, inv_order)
        return gx, gp, None, None
