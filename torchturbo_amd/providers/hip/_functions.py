"""``torch.autograd.Function`` wrappers over the C-ABI kernels.

Each Function allocates its outputs with PyTorch on the input's device and
enqueues the kernels on the current HIP stream. Backward formulas follow
PyTorch autograd of the reference's native compositions:

* permutation (``ops/providers/native/moe_permutation.py:25-57``): token grad =
  fp32 gather-sum of the packed-row grads in ascending row order (the
  ``index_select`` backward); probs grad = packed-probs grad scattered back to
  its (token, expert) cell (the ``masked_select`` backward);
* unpermutation (``:68-99``): unweighted grad = row copy; weighted grad =
  ``cast(grad * w)`` and ``d w = sum_h grad * packed``;
* grouped matmul (``ops/providers/native/grouped_matmul.py:40-53``):
  dX_e = dY_e W_e^T, dW_e = X_e^T dY_e (zero for empty experts), mirrored for
  ``trans_b`` as in ``ops/providers/npu/grouped_matmul.py:41-72``;
* SwiGLU with probabilities and the router top-k: see the kernel sources.
"""

from __future__ import annotations

import torch

from ... import _lib as L
from ... import checks


def require_cuda(*tensors: torch.Tensor | None) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(f"HIP kernels need device tensors; got a tensor on {t.device}.")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError("all tensors must be on the same device")
    return device


def device_counts(counts, num_experts: int, device: torch.device, m: int | None = None) -> torch.Tensor:
    """Per-expert row counts as a contiguous int64 device tensor [E]."""
    if isinstance(counts, torch.Tensor):
        if counts.numel() != num_experts:
            raise ValueError("tokens_per_expert must match the number of expert weight slices.")
        if counts.device.type != "cuda":
            if m is not None and int(counts.sum()) != m:
                raise ValueError(f"tokens_per_expert sums to {int(counts.sum())}, expected {m}")
            return counts.to(device=device, dtype=torch.int64, non_blocking=False).contiguous()
        return counts.to(dtype=torch.int64).contiguous()
    counts = [int(c) for c in counts]
    if len(counts) != num_experts:
        raise ValueError("tokens_per_expert must match the number of expert weight slices.")
    if m is not None and sum(counts) != m:
        raise ValueError(f"tokens_per_expert sums to {sum(counts)}, expected {m}")
    return torch.tensor(counts, dtype=torch.int64, device=device)


# ---------------------------------------------------------------------------
# Router
# ---------------------------------------------------------------------------
class TopKRouting(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, topk, score_function, pre_softmax, num_groups, group_topk,
                scaling_factor, expert_bias, fixed_indices):
        logits = logits.contiguous()
        T, E = logits.shape
        dev = logits.device
        probs = torch.empty_like(logits)
        rmap = torch.empty((T, E), dtype=torch.bool, device=dev)
        top = torch.empty((T, topk), dtype=torch.int64, device=dev)
        bias = None if expert_bias is None else expert_bias.to(device=dev, dtype=torch.float32).contiguous()
        fixed = None if fixed_indices is None else fixed_indices.to(device=dev, dtype=torch.int64).contiguous()
        L.call("tt_router_topk_fwd", L.ptr(logits), L.dtype_code(logits.dtype), T, E, topk,
               L.TT_SCORE[score_function], int(bool(pre_softmax)), L.ptr(bias),
               int(num_groups or 0), int(group_topk or 0), float(scaling_factor or 0.0),
               L.ptr(fixed), L.ptr(probs), L.ptr(rmap), L.ptr(top), L.stream(dev))
        ctx.save_for_backward(logits, top)
        ctx.cfg = (topk, L.TT_SCORE[score_function], int(bool(pre_softmax)), float(scaling_factor or 0.0))
        ctx.mark_non_differentiable(rmap, top)
        # The routing map and indices get no gradient: do not let autograd
        # fill zero tensors for them before every backward.
        ctx.set_materialize_grads(False)
        return probs, rmap, top

    @staticmethod
    def backward(ctx, grad_probs, _g_map, _g_top):
        if grad_probs is None:
            return None, None, None, None, None, None, None, None, None
        logits, top = ctx.saved_tensors
        out = router_topk_bwd(logits, top, grad_probs, *ctx.cfg)
        return out, None, None, None, None, None, None, None, None


def router_topk_bwd(logits, top, grad_probs, topk, sf, pre, scale):
    """d logits of the top-k routing (``tt_router_topk_bwd``), logits dtype."""
    T, E = logits.shape
    grad = grad_probs.to(logits.dtype).contiguous()
    out = torch.empty_like(logits)
    L.call("tt_router_topk_bwd", L.ptr(logits), L.dtype_code(logits.dtype), T, E, topk, sf, pre,
           scale, L.ptr(top), L.ptr(grad), L.ptr(out), L.stream(logits.device))
    return out


class RouterGateTopK(torch.autograd.Function):
    """Gating linear and top-k routing in one kernel (``tt_router_gate_fwd``):
    ``(probs, routing_map, top_indices, logits)`` with ``logits = x W^T`` in
    the router dtype. Backward: the routing gradient (``tt_router_topk_bwd``)
    plus the gradient reaching the logits directly, then the gating linear's
    backward as ``RouterGatingLinearFunction`` forms it (``router.py:44-58``)."""

    @staticmethod
    def forward(ctx, x, weight, router_dtype, topk, score_function, pre_softmax, num_groups,
                group_topk, scaling_factor, expert_bias, fixed_indices):
        x2 = x.reshape(-1, x.shape[-1]).contiguous()
        w = weight.contiguous()
        T, H = x2.shape
        E = w.shape[0]
        dev = x2.device
        logits = torch.empty((T, E), dtype=router_dtype, device=dev)
        probs = torch.empty_like(logits)
        rmap = torch.empty((T, E), dtype=torch.bool, device=dev)
        top = torch.empty((T, topk), dtype=torch.int64, device=dev)
        bias = None if expert_bias is None else expert_bias.to(device=dev, dtype=torch.float32).contiguous()
        fixed = None if fixed_indices is None else fixed_indices.to(device=dev, dtype=torch.int64).contiguous()
        sf = L.TT_SCORE[score_function]
        cfg = (topk, sf, int(bool(pre_softmax)), float(scaling_factor or 0.0))
        L.call("tt_router_gate_fwd", L.ptr(x2), L.ptr(w), L.dtype_code(x2.dtype), T, H, E,
               L.dtype_code(router_dtype), topk, sf, cfg[2], L.ptr(bias), int(num_groups or 0),
               int(group_topk or 0), cfg[3], L.ptr(fixed), L.ptr(logits), L.ptr(probs),
               L.ptr(rmap), L.ptr(top), L.stream(dev))
        ctx.save_for_backward(x2, w, logits, top)
        ctx.cfg = cfg
        ctx.x_shape = x.shape
        ctx.mark_non_differentiable(rmap, top)
        ctx.set_materialize_grads(False)
        return probs, rmap, top, logits

    @staticmethod
    def backward(ctx, g_probs, _g_map, _g_top, g_logits):
        none = (None,) * 9
        x2, w, logits, top = ctx.saved_tensors
        g = None
        if g_probs is not None:
            g = router_topk_bwd(logits, top, g_probs, *ctx.cfg)
        if g_logits is not None:
            g_logits = g_logits.reshape(logits.shape).to(logits.dtype)
            g = g_logits if g is None else g + g_logits
        if g is None:
            return None, None, *none
        rdt = logits.dtype
        gx = gw = None
        if ctx.needs_input_grad[0]:
            gx = g.mm(w.to(rdt)).view(ctx.x_shape).to(x2.dtype)
        if ctx.needs_input_grad[1]:
            gw = g.t().mm(x2.to(rdt)).to(w.dtype)
        return gx, gw, *none


class RouterLossStats(torch.autograd.Function):
    """``(prob_sum [E] f32, tokens_per_expert [E] int64, z_sum [] f32)`` of the
    router logits in one pass (``tt_router_loss_fwd``); the backward is one
    pass too (``tt_router_loss_bwd``). Parts that are switched off come back
    as zeros."""

    @staticmethod
    def forward(ctx, logits, topk, score_function, padding_mask, want_aux, want_z):
        logits = logits.contiguous()
        T, E = logits.shape
        dev = logits.device
        pad = None
        if padding_mask is not None:
            pad = padding_mask.reshape(-1).to(device=dev, dtype=torch.uint8).contiguous()
            if pad.numel() != T:
                raise ValueError(f"padding_mask has {pad.numel()} entries for {T} tokens")
        sf = L.TT_SCORE[score_function]
        if want_aux:
            prob_sum = torch.empty((E,), dtype=torch.float32, device=dev)
            counts = torch.empty((E,), dtype=torch.int64, device=dev)
        else:
            prob_sum = torch.zeros((E,), dtype=torch.float32, device=dev)
            counts = torch.zeros((E,), dtype=torch.int64, device=dev)
        z_sum = (torch.empty if want_z else torch.zeros)((), dtype=torch.float32, device=dev)
        ws_bytes = L.router_loss_workspace(T, E)
        ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
        L.call("tt_router_loss_fwd", L.ptr(logits), L.dtype_code(logits.dtype), T, E, int(topk), sf,
               L.ptr(pad), L.ptr(prob_sum) if want_aux else None,
               L.ptr(counts) if want_aux else None, L.ptr(z_sum) if want_z else None, L.ptr(ws),
               ws_bytes, L.stream(dev))
        ctx.save_for_backward(logits, pad)
        ctx.sf = sf
        ctx.mark_non_differentiable(counts)
        ctx.set_materialize_grads(False)
        return prob_sum, counts, z_sum

    @staticmethod
    def backward(ctx, g_prob_sum, _g_counts, g_z_sum):
        if g_prob_sum is None and g_z_sum is None:
            return None, None, None, None, None, None
        logits, pad = ctx.saved_tensors
        T, E = logits.shape
        gp = None if g_prob_sum is None else g_prob_sum.to(torch.float32).contiguous()
        gz = None if g_z_sum is None else g_z_sum.to(torch.float32).reshape(1).contiguous()
        out = torch.empty_like(logits)
        L.call("tt_router_loss_bwd", L.ptr(logits), L.dtype_code(logits.dtype), T, E, ctx.sf,
               L.ptr(pad), L.ptr(gp), L.ptr(gz), L.ptr(out), L.stream(logits.device))
        return out, None, None, None, None, None


# ---------------------------------------------------------------------------
# Permutation
# ---------------------------------------------------------------------------
def route_index(expert_indices: torch.Tensor, num_experts: int, probs: torch.Tensor | None):
    """Packed-row map of (token, slot) assignments; see ``tt_route_index``."""
    dev = expert_indices.device
    T, K = expert_indices.shape
    ids = expert_indices.to(torch.int64).contiguous()
    rows = torch.empty((T, K), dtype=torch.int32, device=dev)
    token_of_row = torch.empty((T * K,), dtype=torch.int32, device=dev)
    counts = torch.empty((num_experts,), dtype=torch.int64, device=dev)
    packed_probs = None
    pd = None
    if probs is not None:
        pd = probs.contiguous()
        packed_probs = torch.empty((T * K,), dtype=probs.dtype, device=dev)
    ws_bytes = L.route_index_workspace(T, num_experts)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    L.call("tt_route_index", L.ptr(ids), T, max(K, 1), num_experts, L.ptr(pd),
           L.dtype_code(probs.dtype) if probs is not None else 0, L.ptr(rows),
           L.ptr(token_of_row), L.ptr(packed_probs), L.ptr(counts), L.ptr(ws), ws_bytes,
           L.stream(dev))
    if checks.enabled():
        off = L.route_index_rejected_offset(T, num_experts)
        rejected = int(ws[off:off + 4].view(torch.int32).item())
        if rejected:
            raise ValueError(
                f"expert_indices must hold {K} distinct expert ids in [0, {num_experts}) per "
                f"token: {rejected} of {T * K} slots are out of range or repeated."
            )
    return rows, token_of_row, packed_probs, counts


class Permute(torch.autograd.Function):
    @staticmethod
    def forward(ctx, tokens, probs, expert_indices, num_experts):
        ctx.set_materialize_grads(False)  # no zero-filled gradients for rows / counts
        tokens = tokens.contiguous()
        T, H = tokens.shape
        K = expert_indices.shape[1] if expert_indices.dim() == 2 else 0
        dev = tokens.device
        if T == 0 or K == 0:
            rows = torch.empty((T, K), dtype=torch.int32, device=dev)
            counts = torch.zeros((num_experts,), dtype=torch.int64, device=dev)
            packed = tokens.new_empty((0, H))
            pprobs = None if probs is None else probs.new_empty((0,))
            ctx.save_for_backward(rows, expert_indices)
            ctx.shape = (T, H, K, num_experts)
            ctx.mark_non_differentiable(rows, counts)
            return packed, pprobs, rows, counts
        rows, _tor, pprobs, counts = route_index(expert_indices, num_experts, probs)
        packed = tokens.new_empty((T * K, H))
        L.call("tt_permute_scatter", L.ptr(tokens), L.dtype_code(tokens.dtype), T, H, K,
               L.ptr(rows), L.ptr(packed), L.stream(dev))
        ctx.save_for_backward(rows, expert_indices)
        ctx.shape = (T, H, K, num_experts)
        ctx.mark_non_differentiable(rows, counts)
        return packed, pprobs, rows, counts

    @staticmethod
    def backward(ctx, g_packed, g_pprobs, _g_rows, _g_counts):
        rows, experts = ctx.saved_tensors
        T, H, K, E = ctx.shape
        g_tokens = g_probs = None
        if ctx.needs_input_grad[0]:
            if g_packed is None or T == 0 or K == 0:
                g_tokens = torch.zeros((T, H), dtype=g_packed.dtype if g_packed is not None else torch.float32,
                                       device=rows.device)
            else:
                g = g_packed.contiguous()
                g_tokens = g.new_empty((T, H))
                L.call("tt_unpermute_gather", L.ptr(g), L.dtype_code(g.dtype), T, H, K, L.ptr(rows),
                       None, None, 0, max(E, 1), L.ptr(g_tokens), L.stream(g.device))
        if ctx.needs_input_grad[1]:
            if g_pprobs is None or T == 0 or K == 0:
                dt = g_pprobs.dtype if g_pprobs is not None else torch.float32
                g_probs = torch.zeros((T, E), dtype=dt, device=rows.device)
            else:
                gp = g_pprobs.contiguous()
                g_probs = gp.new_empty((T, E))
                L.call("tt_packed_probs_bwd", L.ptr(gp), L.dtype_code(gp.dtype), T, K, E,
                       L.ptr(rows), L.ptr(experts.to(torch.int64).contiguous()), L.ptr(g_probs),
                       L.stream(gp.device))
        return g_tokens, g_probs, None, None


class Unpermute(torch.autograd.Function):
    @staticmethod
    def forward(ctx, packed, rows, experts, probs, num_tokens):
        packed = packed.contiguous()
        H = packed.shape[1]
        T = num_tokens
        K = rows.shape[1] if rows.dim() == 2 else 0
        dev = packed.device
        rows = rows.to(torch.int32).contiguous()
        experts = experts.to(torch.int64).contiguous()
        out = packed.new_empty((T, H))
        E = probs.shape[1] if probs is not None else 1
        if T > 0 and K > 0:
            pc = probs.contiguous() if probs is not None else None
            L.call("tt_unpermute_gather", L.ptr(packed), L.dtype_code(packed.dtype), T, H, K,
                   L.ptr(rows), L.ptr(experts), L.ptr(pc),
                   L.dtype_code(probs.dtype) if probs is not None else 0, E, L.ptr(out),
                   L.stream(dev))
        elif T > 0:
            out.zero_()
        if probs is not None:
            ctx.save_for_backward(rows, experts, packed, probs)
        else:
            ctx.save_for_backward(rows, experts)
        ctx.meta = (T, H, K, probs is not None, packed.shape[0])
        return out

    @staticmethod
    def backward(ctx, g_out):
        T, H, K, weighted, M = ctx.meta
        g = g_out.contiguous()
        if weighted:
            rows, experts, packed, probs = ctx.saved_tensors
        else:
            rows, experts = ctx.saved_tensors
        g_packed = g.new_zeros((M, H)) if (T == 0 or K == 0) else g.new_empty((M, H))
        g_probs = None
        if T == 0 or K == 0:
            if weighted:
                g_probs = torch.zeros_like(probs)
            return g_packed, None, None, g_probs, None
        dev = g.device
        if not weighted:
            L.call("tt_permute_scatter", L.ptr(g), L.dtype_code(g.dtype), T, H, K, L.ptr(rows),
                   L.ptr(g_packed), L.stream(dev))
        else:
            pc = probs.contiguous()
            g_probs = torch.empty_like(pc)
            L.call("tt_unpermute_gather_bwd", L.ptr(g), L.ptr(packed), L.dtype_code(g.dtype), T, H, K,
                   L.ptr(rows), L.ptr(experts), L.ptr(pc), L.dtype_code(pc.dtype), pc.shape[1],
                   L.ptr(g_packed), L.ptr(g_probs), L.stream(dev))
        return g_packed, None, None, g_probs, None


# ---------------------------------------------------------------------------
# SwiGLU (+ probability weighting)
# ---------------------------------------------------------------------------
class SwiGLU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, probs):
        x = x.contiguous()
        rows, two_f = x.shape
        if two_f % 2:
            raise ValueError("swiglu expects an even last dimension")
        F = two_f // 2
        out = x.new_empty((rows, F))
        pc = probs.contiguous() if probs is not None else None
        L.call("tt_swiglu_fwd", L.ptr(x), L.dtype_code(x.dtype), rows, F, L.ptr(pc),
               L.dtype_code(probs.dtype) if probs is not None else 0, L.ptr(out), L.stream(x.device))
        ctx.save_for_backward(x, pc)
        return out

    @staticmethod
    def backward(ctx, g_out):
        x, probs = ctx.saved_tensors
        rows, two_f = x.shape
        g = g_out.to(x.dtype).contiguous()
        gx = torch.empty_like(x)
        gp = None
        if probs is not None and ctx.needs_input_grad[1]:
            gp = torch.empty_like(probs)
        L.call("tt_swiglu_bwd", L.ptr(x), L.dtype_code(x.dtype), rows, two_f // 2, L.ptr(probs),
               L.dtype_code(probs.dtype) if probs is not None else 0, L.ptr(g), L.ptr(gx),
               L.ptr(gp), L.stream(x.device))
        return gx, gp


class GatedActivation(torch.autograd.Function):
    """act(gate) * up with an optional cap, and the probability product
    (``tt_gated_act_fwd`` / ``tt_gated_act_bwd``); act 0 = SiLU, 1 = GELU."""

    @staticmethod
    def forward(ctx, x, probs, act, limit, clamp_after):
        x = x.contiguous()
        rows, two_f = x.shape
        if two_f % 2:
            raise ValueError("gated_activation expects an even last dimension")
        F = two_f // 2
        out = x.new_empty((rows, F))
        pc = probs.contiguous() if probs is not None else None
        L.call("tt_gated_act_fwd", L.ptr(x), L.dtype_code(x.dtype), rows, F, int(act),
               float(limit), int(bool(clamp_after)), L.ptr(pc),
               L.dtype_code(probs.dtype) if probs is not None else 0, L.ptr(out),
               L.stream(x.device))
        ctx.save_for_backward(x, pc)
        ctx.cfg = (int(act), float(limit), int(bool(clamp_after)))
        return out

    @staticmethod
    def backward(ctx, g_out):
        x, probs = ctx.saved_tensors
        act, limit, after = ctx.cfg
        rows, two_f = x.shape
        g = g_out.to(x.dtype).contiguous()
        gx = torch.empty_like(x)
        gp = None
        if probs is not None and ctx.needs_input_grad[1]:
            gp = torch.empty_like(probs)
        L.call("tt_gated_act_bwd", L.ptr(x), L.dtype_code(x.dtype), rows, two_f // 2, act, limit,
               after, L.ptr(probs), L.dtype_code(probs.dtype) if probs is not None else 0,
               L.ptr(g), L.ptr(gx), L.ptr(gp), L.stream(x.device))
        return gx, gp, None, None, None


# ---------------------------------------------------------------------------
# Grouped GEMM
# ---------------------------------------------------------------------------
class GroupedMatmul(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, counts, trans_b):
        x = x.contiguous()
        w = w.contiguous()
        E = w.shape[0]
        M, K = x.shape
        N = w.shape[1] if trans_b else w.shape[2]
        kw = w.shape[2] if trans_b else w.shape[1]
        if kw != K:
            raise ValueError(f"grouped_matmul: x has {K} features, weight expects {kw}")
        if x.dtype != w.dtype:
            raise ValueError("grouped_matmul: x and weight dtypes differ")
        y = x.new_empty((M, N))
        if M > 0:
            L.call("tt_gmm_fwd", L.ptr(x), L.ptr(w), L.dtype_code(x.dtype), M, K, N, E, int(trans_b),
                   L.ptr(counts), L.ptr(y), L.stream(x.device))
        ctx.save_for_backward(x, w, counts)
        ctx.trans_b = bool(trans_b)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, counts = ctx.saved_tensors
        tb = ctx.trans_b
        dy = dy.to(x.dtype).contiguous()
        E = w.shape[0]
        M, K = x.shape
        N = dy.shape[1]
        dx = dw = None
        dev = x.device
        if ctx.needs_input_grad[0]:
            dx = x.new_empty((M, K))
            if M > 0:
                L.call("tt_gmm_dgrad", L.ptr(dy), L.ptr(w), L.dtype_code(x.dtype), M, K, N, E, int(tb),
                       L.ptr(counts), L.ptr(dx), L.stream(dev))
        if ctx.needs_input_grad[1]:
            dw = torch.empty_like(w)
            L.call("tt_gmm_wgrad", L.ptr(x), L.ptr(dy), L.dtype_code(x.dtype), M, K, N, E, int(tb),
                   L.ptr(counts), L.ptr(dw), L.stream(dev))
        return dx, dw, None, None


class GroupedMatmulFp8(torch.autograd.Function):
    """y = x @ deq(qw[e])^T; the weight gradient goes to ``master`` ([E, N, K])."""

    @staticmethod
    def forward(ctx, x, master, qw, scale, counts):
        x = x.contiguous()
        qw = qw.contiguous()
        scale = scale.contiguous()
        E, N, K = qw.shape
        M = x.shape[0]
        if x.shape[1] != K:
            raise ValueError(f"grouped_matmul_fp8: x has {x.shape[1]} features, weight expects {K}")
        if x.dtype != torch.bfloat16:
            raise ValueError("grouped_matmul_fp8: activations must be bf16")
        y = x.new_empty((M, N))
        if M > 0:
            L.call("tt_gmm_fp8_fwd", L.ptr(x), L.ptr(qw), L.ptr(scale), L.dtype_code(scale.dtype),
                   M, K, N, E, L.ptr(counts), L.ptr(y), L.stream(x.device))
        ctx.save_for_backward(x, qw, scale, counts)
        ctx.has_master = master is not None
        return y

    @staticmethod
    def backward(ctx, dy):
        x, qw, scale, counts = ctx.saved_tensors
        dy = dy.to(torch.bfloat16).contiguous()
        E, N, K = qw.shape
        M = x.shape[0]
        dev = x.device
        dx = dmaster = None
        if ctx.needs_input_grad[0]:
            dx = x.new_empty((M, K))
            if M > 0:
                L.call("tt_gmm_fp8_dgrad", L.ptr(dy), L.ptr(qw), L.ptr(scale), L.dtype_code(scale.dtype),
                       M, K, N, E, L.ptr(counts), L.ptr(dx), L.stream(dev))
        if ctx.has_master and ctx.needs_input_grad[1]:
            dmaster = torch.empty((E, N, K), dtype=torch.bfloat16, device=dev)
            L.call("tt_gmm_wgrad", L.ptr(x), L.ptr(dy), L.TT_BF16, M, K, N, E, 1, L.ptr(counts),
                   L.ptr(dmaster), L.stream(dev))
        return dx, dmaster, None, None, None
