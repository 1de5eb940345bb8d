"""The CPU oracle layer evaluated on part of a full-size workload.

At the configurations' real sizes (Mixtral 8192 x 4096 x 14336, DeepSeek-V3
with 256 FP8 experts of 7168 x 2048, the 72k-token varlen batch) the oracle
cannot run the whole layer in seconds, but it does not need to:

* each row of the output, of d_hidden and of d_logits depends only on its own
  token: its logits row, its hidden row, its grad row and the weights of the
  experts it is routed to. ``token_rows`` runs the oracle on a token subset
  with only the experts that subset uses (experts renumbered in order, which
  keeps the expert-major packed order);
* the weight gradient of expert e depends only on the tokens routed to e and
  on expert e's own term of the layer sum (the output gradient is given, and
  the unweighted combine passes each packed row its token's gradient row),
  and the gate / up columns c of dW1[e] and the rows c of dW2[e] only on the
  ffn columns c (SwiGLU is elementwise). ``expert_grads`` runs the oracle's
  expert terms (grouped matmul, SwiGLU x probability, grouped matmul) of the
  chosen experts on every token routed to them, on an ffn column slice, and
  returns those experts' gradients on that slice; no other expert is
  evaluated, so the most-loaded expert of a full-size layer stays cheap.

Both results equal the rows / slices of the full oracle run up to the
summation order of CPU matrix products (``test_sampled_oracle_matches_full``).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from oracle import layer as o_layer
from oracle.fp8 import dequantize_experts


@dataclass
class ExpertWeights:
    """Full expert weights on the CPU: bf16 ``w1 [E, H, 2F]`` / ``w2 [E, F, H]``,
    or FP8 ``q1 [E, 2F, H]``, ``s1``, ``q2 [E, H, F]``, ``s2`` (HF [out, in])."""

    w1: torch.Tensor | None = None
    w2: torch.Tensor | None = None
    q1: torch.Tensor | None = None
    s1: torch.Tensor | None = None
    q2: torch.Tensor | None = None
    s2: torch.Tensor | None = None
    getter: object = None  # optional callable(experts, f_slice) -> ExpertWeights (lazy fetch)

    @property
    def fp8(self) -> bool:
        return self.q1 is not None

    def select(self, experts: torch.Tensor, f_slice: tuple[int, int] | None):
        """Weights of ``experts`` (sorted ids), ffn columns ``f_slice`` (or all)."""
        if self.getter is not None:
            return self.getter(experts, f_slice)
        every = self.q1 if self.fp8 else self.w1
        if f_slice is None and experts.numel() == every.shape[0]:
            return self  # sorted and complete: every expert, in order (no copy)
        if not self.fp8:
            w1, w2 = self.w1[experts], self.w2[experts]
            if f_slice is not None:
                c0, c1 = f_slice
                F = w2.shape[1]
                w1 = torch.cat([w1[:, :, c0:c1], w1[:, :, F + c0:F + c1]], dim=2)
                w2 = w2[:, c0:c1]
            return ExpertWeights(w1=w1.contiguous(), w2=w2.contiguous())
        q1, s1, q2, s2 = self.q1[experts], self.s1[experts], self.q2[experts], self.s2[experts]
        if f_slice is not None:
            c0, c1 = f_slice
            assert c0 % 128 == 0 and c1 % 128 == 0, "FP8 slices follow the 128 scale blocks"
            F = q2.shape[2]
            b0, b1, bF = c0 // 128, c1 // 128, F // 128
            q1 = torch.cat([q1[:, c0:c1], q1[:, F + c0:F + c1]], dim=1)
            s1 = torch.cat([s1[:, b0:b1], s1[:, bF + b0:bF + b1]], dim=1)
            q2, s2 = q2[:, :, c0:c1], s2[:, :, b0:b1]
        return ExpertWeights(q1=q1.contiguous(), s1=s1.contiguous(), q2=q2.contiguous(),
                             s2=s2.contiguous())


@dataclass
class SampleResult:
    tokens: torch.Tensor          # token ids of the rows below
    out: torch.Tensor             # [n, H]
    d_hidden: torch.Tensor        # [n, H]
    d_logits: torch.Tensor        # [n, E]
    expert_indices: torch.Tensor  # [n, k] (original expert ids)
    d_w1: dict                    # expert id -> [H, 2f] (bf16 layout) or [2f, H] (FP8 layout)
    d_w2: dict                    # expert id -> [f, H] or [H, f]


def _run(hidden, logits, grad, cfg, bias, weights: ExpertWeights, tokens, f_slice, shared,
         weight_grads=True):
    E = logits.shape[1]
    hr = hidden[tokens].clone().requires_grad_()
    lr = logits[tokens].clone().requires_grad_()
    probs, rmap, ids = o_layer.route(lr, cfg, bias)
    used = rmap.any(dim=0).nonzero().flatten()
    renum = torch.full((E,), -1, dtype=torch.long)
    renum[used] = torch.arange(used.numel())
    sel = weights.select(used, f_slice)
    if sel.fp8:
        m1 = dequantize_experts(sel.q1, sel.s1).requires_grad_(weight_grads)
        m2 = dequantize_experts(sel.q2, sel.s2).requires_grad_(weight_grads)
        fp8 = {"q1": sel.q1, "s1": sel.s1, "q2": sel.q2, "s2": sel.s2, "m1": m1, "m2": m2}
        w1 = w2 = None
        g1, g2 = m1, m2
    else:
        fp8 = None
        w1 = sel.w1.detach().requires_grad_(weight_grads)  # shares storage; nothing writes it
        w2 = sel.w2.detach().requires_grad_(weight_grads)
        g1, g2 = w1, w2
    out = o_layer.moe_layer_routed(hr, probs[:, used], rmap[:, used], renum[ids], w1, w2,
                                   fp8=fp8, shared=shared, stacked_grad=True)
    out.backward(grad[tokens])
    d_w1 = {int(e): g1.grad[i] for i, e in enumerate(used.tolist())} if weight_grads else {}
    d_w2 = {int(e): g2.grad[i] for i, e in enumerate(used.tolist())} if weight_grads else {}
    return SampleResult(tokens, out.detach(), hr.grad, lr.grad, ids, d_w1, d_w2)


def token_rows(hidden, logits, grad, cfg, bias, weights: ExpertWeights, tokens, shared=None):
    """Oracle output, d_hidden and d_logits rows of ``tokens`` (full ffn; no
    weight gradients)."""
    return _run(hidden, logits, grad, cfg, bias, weights, tokens, None, shared,
                weight_grads=False)


def expert_grads(hidden, logits, grad, cfg, bias, weights: ExpertWeights, experts,
                 f_slice=None, full_ids=None):
    """Weight gradients of ``experts`` on the ffn columns ``f_slice``.

    ``full_ids`` [T, k]: the routing of all tokens (the oracle's, or any exact
    equal), used to find every token routed to the chosen experts."""
    if full_ids is None:
        full_ids = o_layer.route(logits, cfg, bias)[2]
    E = logits.shape[1]
    chosen = sorted({int(e) for e in experts})
    mask = torch.zeros(E, dtype=torch.bool)
    mask[chosen] = True
    tokens = mask[full_ids].any(dim=1).nonzero().flatten()
    probs, rmap, _ = o_layer.route(logits[tokens], cfg, bias)
    # Packed rows of the chosen experts: experts ascending, tokens ascending
    # (the permutation's order restricted to these experts).
    sub = rmap[:, chosen]
    counts = sub.sum(dim=0).long()
    cell = sub.t().contiguous().reshape(-1).nonzero().flatten()
    row_token = cell % max(tokens.numel(), 1)
    row_expert = cell // max(tokens.numel(), 1)
    x = hidden[tokens][row_token]
    p = probs[:, chosen].t().reshape(-1)[cell]
    g_rows = grad[tokens][row_token]
    sel = weights.select(torch.tensor(chosen), f_slice)
    if sel.fp8:
        m1 = dequantize_experts(sel.q1, sel.s1).requires_grad_()
        m2 = dequantize_experts(sel.q2, sel.s2).requires_grad_()
        fc1 = o_layer.grouped_matmul_fp8(x, sel.q1, sel.s1, counts, master=m1, stacked_grad=True)
        act = o_layer.swiglu_probs(fc1, p)
        fc2 = o_layer.grouped_matmul_fp8(act, sel.q2, sel.s2, counts, master=m2,
                                         stacked_grad=True)
        g1, g2 = m1, m2
    else:
        g1 = sel.w1.detach().requires_grad_()  # shares storage; nothing writes it
        g2 = sel.w2.detach().requires_grad_()
        fc1 = o_layer.grouped_matmul(x, g1, counts, stacked_grad=True)
        act = o_layer.swiglu_probs(fc1, p)
        fc2 = o_layer.grouped_matmul(act, g2, counts, stacked_grad=True)
    fc2.backward(g_rows.to(fc2.dtype))
    assert torch.equal(row_expert.bincount(minlength=len(chosen)), counts)
    d_w1 = {e: g1.grad[i] for i, e in enumerate(chosen)}
    d_w2 = {e: g2.grad[i] for i, e in enumerate(chosen)}
    empty = torch.empty(0)
    return SampleResult(tokens, empty, empty, empty, full_ids[tokens], d_w1, d_w2)


__all__ = ["ExpertWeights", "SampleResult", "expert_grads", "token_rows"]
