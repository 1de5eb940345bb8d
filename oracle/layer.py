"""The reference MoE layer composition on the CPU (oracle).

Restates the EP=1 data flow of ``MoELayer.forward``
(``src/torchturbo/models/modules/moe/moe_layer.py:149-183``):

1. routing (``router.py:277-356`` -> ``utils.py:127-230``), from given logits;
2. ``dispatch_preprocess`` (``token_dispatcher.py:149-176``): per-expert
   counts ``routing_map.sum(0)`` and the mask permutation with probs;
3. EP=1: the all-to-all is the identity (``comm.py:147-150``) and the chunk
   sort uses the identity order (``token_dispatcher.py:101-107``);
4. ``GroupedMLP.forward`` (``experts.py:188-266``): fc1 grouped matmul,
   SwiGLU, probability weighting in the probs dtype, fc2 grouped matmul;
5. ``combine_postprocess`` (``token_dispatcher.py:222-236``): unweighted
   unpermutation, then ``.to(hidden.dtype)``;
6. shared experts are added last (``moe_layer.py:181-182``).

The FP8 variant replaces both grouped matmuls by the dequantize-then-BF16
composition of ``native_providers/grouped_matmul_fp8.py``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from torchturbo_amd.dispatch import MoEPermutation

from .native_providers.grouped_matmul import grouped_matmul
from .native_providers.grouped_matmul_fp8 import grouped_matmul_fp8
from .native_providers.moe_permutation import permute, unpermute
from .native_providers.routing import topk_softmax_with_capacity
from .native_providers.swiglu import swiglu_probs


@dataclass
class RoutingConfig:
    topk: int
    pre_softmax: bool = False
    score_function: str = "softmax"
    num_groups: int | None = None
    group_topk: int | None = None
    scaling_factor: float | None = None


@dataclass
class LayerTrace:
    probs: torch.Tensor
    routing_map: torch.Tensor
    expert_indices: torch.Tensor
    tokens_per_expert: torch.Tensor
    permutation: MoEPermutation
    fc1: torch.Tensor
    act: torch.Tensor
    fc2: torch.Tensor


def route(logits, cfg: RoutingConfig, expert_bias=None):
    return topk_softmax_with_capacity(
        logits, cfg.topk, use_pre_softmax=cfg.pre_softmax, num_groups=cfg.num_groups,
        group_topk=cfg.group_topk, scaling_factor=cfg.scaling_factor,
        score_function=cfg.score_function, expert_bias=expert_bias,
    )


def moe_layer(hidden, logits, w1, w2, cfg: RoutingConfig, *, expert_bias=None,
              shared=None, fp8=None, trace: bool = False):
    """hidden [T, H]; logits [T, E]; w1 [E, H, 2F]; w2 [E, F, H].

    ``fp8``: optional dict with ``q1, s1, q2, s2`` (HF [out, in] orientation:
    q1 [E, 2F, H], q2 [E, H, F]) and optional ``m1, m2`` gradient sinks; when
    given, ``w1``/``w2`` are ignored. ``shared``: optional callable on hidden.
    """
    probs, routing_map, ids = route(logits, cfg, expert_bias)
    return moe_layer_routed(hidden, probs, routing_map, ids, w1, w2, shared=shared, fp8=fp8,
                            trace=trace)


def moe_layer_routed(hidden, probs, routing_map, ids, w1, w2, *, shared=None, fp8=None,
                     trace: bool = False, stacked_grad: bool = False):
    """Steps 2-6 from a routing result: probs [T, E], routing_map [T, E] (bool),
    ids [T, k]. Every output row depends only on its own token's routing, so a
    caller may pass a subset of the tokens, and only the experts that subset
    uses (columns of probs / routing_map, ids renumbered in the same order).
    ``stacked_grad``: see ``native_providers.grouped_matmul.grouped_matmul``."""
    counts = routing_map.sum(dim=0).long()
    perm = permute(hidden, routing_map, probs=probs, expert_indices=ids)
    sg = dict(stacked_grad=stacked_grad)
    if fp8 is None:
        fc1 = grouped_matmul(perm.tokens, w1, counts, **sg)
    else:
        fc1 = grouped_matmul_fp8(perm.tokens, fp8["q1"], fp8["s1"], counts, master=fp8.get("m1"),
                                 **sg)
    act = swiglu_probs(fc1, perm.probs)
    if fp8 is None:
        fc2 = grouped_matmul(act, w2, counts, **sg)
    else:
        fc2 = grouped_matmul_fp8(act, fp8["q2"], fp8["s2"], counts, master=fp8.get("m2"), **sg)
    combined = unpermute(
        MoEPermutation(fc2, None, perm.row_indices, perm.expert_indices), hidden.shape
    )
    out = combined.to(hidden.dtype)
    if shared is not None:
        out = out + shared(hidden)
    if trace:
        return out, LayerTrace(probs, routing_map, ids, counts, perm, fc1, act, fc2)
    return out


def dense_mlp(hidden, gate_w, up_w, down_w):
    """HF dense SwiGLU MLP (shared expert): ``down(silu(gate(x)) * up(x))``."""
    return F.linear(F.silu(F.linear(hidden, gate_w)) * F.linear(hidden, up_w), down_w)
