"""Expert MLP with the permutation and unpermutation folded into its GEMMs.

On one GPU holding every expert, the layer's token path is

    permute (x -> packed rows) -> fc1 -> activation -> fc2 -> unpermute (sum rows per token)

(``models/modules/moe/token_dispatcher.py:80-259`` around ``experts.py:188-266``).
The packed copies of the tokens (forward) and of the output gradient (the
backward of the unpermutation) exist only to be read by one GEMM each and by a
weight gradient. Here those GEMMs read their rows straight from the token
matrices through the routing index's ``token_of_row`` map
(``tt_gmm_fwd_gather`` / ``tt_gmm_dgrad_gather`` / ``tt_gmm_wgrad_gather``), so
neither copy is written or read: two passes of T·k·H·2 bytes each way fewer per
step. Every GEMM sees the same operand values in the same order as the packed
path, so outputs and gradients are bit-identical to
permute + ``GroupedMLP`` + unpermute.

Used by ``MoELayer`` when the HIP providers serve the three ops, the experts are
a bf16 / f16 ``GroupedMLP`` without ``moe_apply_probs_on_input``, the hidden
size is a multiple of 64 above 64, the experts average more than 512 rows (the
weight-gradient kernel that gathers) and fc1 is at most twice as wide as the
hidden size (see ``eligible``). ``TORCHTURBO_AMD_FUSED_PERMUTE=0`` turns it off.
"""

from __future__ import annotations

import os

import torch

from ... import _lib as L
from ... import checks
from ._functions import route_index
from .moe_permutation import _check_map_matches_indices


class RoutePacked(torch.autograd.Function):
    """Routing index and probs in packed order; the probs' gradient flows back
    through ``tt_packed_probs_bwd`` (the masked_select backward of
    ``native/moe_permutation.py:44-46``)."""

    @staticmethod
    def forward(ctx, probs, expert_indices, num_experts):
        ctx.set_materialize_grads(False)
        rows, token_of_row, pprobs, counts = route_index(expert_indices, num_experts, probs)
        ctx.save_for_backward(rows, expert_indices)
        ctx.num_experts = num_experts
        ctx.mark_non_differentiable(rows, token_of_row, counts)
        return pprobs, rows, token_of_row, counts

    @staticmethod
    def backward(ctx, g_pprobs, _g_rows, _g_tor, _g_counts):
        rows, experts = ctx.saved_tensors
        T, K = rows.shape
        E = ctx.num_experts
        if g_pprobs is None:
            return None, None, None
        gp = g_pprobs.contiguous()
        g_probs = gp.new_empty((T, E))
        L.call("tt_packed_probs_bwd", L.ptr(gp), L.dtype_code(gp.dtype), T, K, E, L.ptr(rows),
               L.ptr(experts.to(torch.int64).contiguous()), L.ptr(g_probs), L.stream(gp.device))
        return g_probs, None, None


class GatherGroupedMatmul(torch.autograd.Function):
    """y[r] = tokens[token_of_row[r]] @ W[e(r)]: the permutation and fc1 in one
    launch. Backward: the packed data gradient summed back onto its tokens (the
    permutation's backward, ``tt_unpermute_gather`` without weights) and the
    weight gradient gathering the token rows."""

    @staticmethod
    def forward(ctx, tokens, w, counts, rows, token_of_row, trans_b):
        tokens = tokens.contiguous()
        w = w.contiguous()
        T, K = tokens.shape
        M = token_of_row.shape[0]
        E = w.shape[0]
        N = w.shape[1] if trans_b else w.shape[2]
        y = tokens.new_empty((M, N))
        if M > 0:
            L.call("tt_gmm_fwd_gather", L.ptr(tokens), T, L.ptr(token_of_row), L.ptr(w),
                   L.dtype_code(tokens.dtype), M, K, N, E, int(trans_b), L.ptr(counts), L.ptr(y),
                   L.stream(tokens.device))
        ctx.save_for_backward(tokens, w, counts, rows, token_of_row)
        ctx.trans_b = bool(trans_b)
        return y

    @staticmethod
    def backward(ctx, dy):
        tokens, w, counts, rows, token_of_row = ctx.saved_tensors
        tb = ctx.trans_b
        dy = dy.to(tokens.dtype).contiguous()
        T, K = tokens.shape
        M, N = dy.shape
        E = w.shape[0]
        dev = tokens.device
        code = L.dtype_code(tokens.dtype)
        d_tokens = dw = None
        if ctx.needs_input_grad[0]:
            d_packed = tokens.new_empty((M, K))
            d_tokens = tokens.new_empty((T, K))
            if M > 0:
                L.call("tt_gmm_dgrad", L.ptr(dy), L.ptr(w), code, M, K, N, E, int(tb),
                       L.ptr(counts), L.ptr(d_packed), L.stream(dev))
            L.call("tt_unpermute_gather", L.ptr(d_packed), code, T, K, rows.shape[1],
                   L.ptr(rows), None, None, 0, max(E, 1), L.ptr(d_tokens), L.stream(dev))
        if ctx.needs_input_grad[1]:
            dw = torch.empty_like(w)
            L.call("tt_gmm_wgrad_gather", L.ptr(tokens), T, L.ptr(token_of_row), L.ptr(dy), 0,
                   None, code, M, K, N, E, int(tb), L.ptr(counts), L.ptr(dw), L.stream(dev))
        return d_tokens, dw, None, None, None, None


class GroupedMatmulCombine(torch.autograd.Function):
    """out[t] = sum over the token's rows r of (act[r] @ W[e(r)]): fc2 and the
    unweighted unpermutation. Backward: the output gradient's rows are gathered
    per packed row inside the data and weight gradients (the unpermutation's
    backward copy, ``tt_permute_scatter``, is never made)."""

    @staticmethod
    def forward(ctx, act, w, counts, rows, token_of_row, trans_b):
        act = act.contiguous()
        w = w.contiguous()
        M, K = act.shape
        T, topk = rows.shape
        E = w.shape[0]
        N = w.shape[1] if trans_b else w.shape[2]
        dev = act.device
        code = L.dtype_code(act.dtype)
        y = act.new_empty((M, N))
        if M > 0:
            L.call("tt_gmm_fwd", L.ptr(act), L.ptr(w), code, M, K, N, E, int(trans_b),
                   L.ptr(counts), L.ptr(y), L.stream(dev))
        out = act.new_empty((T, N))
        L.call("tt_unpermute_gather", L.ptr(y), code, T, N, topk, L.ptr(rows), None, None, 0,
               max(E, 1), L.ptr(out), L.stream(dev))
        ctx.save_for_backward(act, w, counts, token_of_row)
        ctx.trans_b = bool(trans_b)
        return out

    @staticmethod
    def backward(ctx, d_out):
        act, w, counts, token_of_row = ctx.saved_tensors
        tb = ctx.trans_b
        d_out = d_out.to(act.dtype).contiguous()
        M, K = act.shape
        T, N = d_out.shape
        E = w.shape[0]
        dev = act.device
        code = L.dtype_code(act.dtype)
        d_act = dw = None
        if ctx.needs_input_grad[0]:
            d_act = act.new_empty((M, K))
            if M > 0:
                L.call("tt_gmm_dgrad_gather", L.ptr(d_out), T, L.ptr(token_of_row), L.ptr(w), code,
                       M, K, N, E, int(tb), L.ptr(counts), L.ptr(d_act), L.stream(dev))
        if ctx.needs_input_grad[1]:
            dw = torch.empty_like(w)
            L.call("tt_gmm_wgrad_gather", L.ptr(act), 0, None, L.ptr(d_out), T,
                   L.ptr(token_of_row), code, M, K, N, E, int(tb), L.ptr(counts), L.ptr(dw),
                   L.stream(dev))
        return d_act, dw, None, None, None, None


def enabled() -> bool:
    return os.environ.get("TORCHTURBO_AMD_FUSED_PERMUTE", "1") != "0"


def eligible(tokens: torch.Tensor, w1: torch.Tensor, topk: int, num_experts: int) -> bool:
    """Shapes and dtypes the gathering kernels cover (see the module docstring),
    where gathering pays: fc1's output at most twice the hidden size. The two
    passes saved scale with T·k·H, the cost of gathering inside the long weight
    gradients with their work, T·k·H·F: on Qwen3-30B-A3B (F 768, H 2048) the
    layer step is 4 % faster, on Mixtral (F 14336, H 4096) it would be 1-3 %
    slower (its weight gradients re-read each gathered row slice many times)."""
    if not enabled() or not tokens.is_cuda or tokens.dim() != 2 or w1.dtype != tokens.dtype:
        return False
    T, H = tokens.shape
    return shapes_pay(T, H, w1.shape[-1], topk, num_experts, tokens.dtype)


def shapes_pay(tokens: int, hidden: int, fc1_width: int, topk: int, num_experts: int,
               dtype: torch.dtype) -> bool:
    """The shape part of ``eligible``: fc1 at most twice as wide as the hidden
    size (where gathering pays), and every gathering GEMM of the layer takes
    the shapes, as the library reports without launching
    (``tt_gmm_gather_supported``): fc1 forward with gathered token rows
    ([T, H] source, reduction H), fc1's weight gradient with gathered x rows,
    fc2's data gradient with gathered output-gradient rows (reduction H) and
    fc2's weight gradient with gathered output-gradient rows (more than 512
    routed rows per expert on average, 16-bit, reductions a multiple of 64
    above 64, the experts' schedule in LDS)."""
    if dtype not in (torch.bfloat16, torch.float16) or fc1_width > 2 * hidden:
        return False
    lib = L.load()
    code = L.dtype_code(dtype)
    m = tokens * topk
    ffn = fc1_width // 2
    return all(lib.tt_gmm_gather_supported(op, code, tokens, m, k, n, num_experts) == 1
               for op, k, n in ((0, hidden, fc1_width), (2, hidden, fc1_width),
                                (1, ffn, hidden), (3, ffn, hidden)))


def grouped_mlp_tokens(experts, tokens, probs, routing_map, expert_indices):
    """``GroupedMLP`` over the tokens a routing selects, summed back per token:
    the output and gradients of permute -> experts -> unpermute. Returns the
    output [T, H] and the per-expert counts (int64, on the device)."""
    cfg = experts.config
    E = experts.num_local_experts
    H = cfg.hidden_size
    pprobs, rows, token_of_row, counts = RoutePacked.apply(probs, expert_indices, E)
    if checks.enabled():  # after the id check inside the routing index
        _check_map_matches_indices(routing_map, expert_indices)
    w1 = experts.weight1.view(E, H, -1)
    w2 = experts.weight2.view(E, -1, H)
    fc1 = GatherGroupedMatmul.apply(tokens, w1, counts, rows, token_of_row, False)
    act = experts.activation_func_with_probs(fc1, pprobs)
    return GroupedMatmulCombine.apply(act, w2, counts, rows, token_of_row, False), counts
