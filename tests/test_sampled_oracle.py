"""The sampled oracle (``tests/sampled_oracle.py``) against the full oracle run.

The full-size GPU layer tests check token rows and per-expert weight-gradient
slices against the oracle evaluated on a token subset. This pins that
decomposition on the CPU: on small layers where the whole oracle runs, the
subset results equal the full run's rows and slices (fp32: to the summation
order of CPU matrix products; the FP8 path is bf16 throughout).
"""

from __future__ import annotations

from dataclasses import replace

import pytest
import torch

from oracle import layer as o_layer
from oracle.fp8 import dequantize_experts
from tests.conftest import assert_bf16_close, rel_errors
from tests.sampled_oracle import ExpertWeights, expert_grads, token_rows
from torchturbo_amd import configs as C


def _cfg(w):
    return o_layer.RoutingConfig(topk=w.topk, pre_softmax=w.pre_softmax,
                                 score_function=w.score_function, num_groups=w.num_groups,
                                 group_topk=w.group_topk, scaling_factor=w.scaling_factor)


def _close(a, b, fp32, what):
    if fp32:
        mx, _ = rel_errors(a, b)
        assert mx <= 1e-5, (what, mx)
    else:
        assert_bf16_close(a, b, what=what)


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16_layout_fp32", "fp8"])
def test_sampled_oracle_matches_full(fp8):
    if fp8:
        w = replace(C.DSV3, tokens=192, hidden=256, ffn=256, experts=16, num_groups=4,
                    group_topk=2, shared_ffn=None)
    else:
        w = replace(C.QWEN3, tokens=192, hidden=128, ffn=96, experts=16, topk=4,
                    dtype=torch.float32)
    hidden, logits, grad = C.make_hidden(w), C.make_logits(w), C.make_grad(w)
    bias = C.make_expert_bias(w)
    m1, m2 = C.make_weights(w)
    cfg = _cfg(w)
    if fp8:
        q1, s1 = C.fp8_blocks(m1.transpose(1, 2).contiguous())
        q2, s2 = C.fp8_blocks(m2.transpose(1, 2).contiguous())
        weights = ExpertWeights(q1=q1, s1=s1, q2=q2, s2=s2)
        d1 = dequantize_experts(q1, s1).requires_grad_()
        d2 = dequantize_experts(q2, s2).requires_grad_()
        fp8d = {"q1": q1, "s1": s1, "q2": q2, "s2": s2, "m1": d1, "m2": d2}
        w1r = w2r = None
        g1, g2 = d1, d2
    else:
        weights = ExpertWeights(w1=m1, w2=m2)
        w1r, w2r = m1.clone().requires_grad_(), m2.clone().requires_grad_()
        fp8d = None
        g1, g2 = w1r, w2r
    hr, lr = hidden.clone().requires_grad_(), logits.clone().requires_grad_()
    out, trace = o_layer.moe_layer(hr, lr, w1r, w2r, cfg, expert_bias=bias, fp8=fp8d, trace=True)
    out.backward(grad)
    fp32 = not fp8

    tokens = torch.tensor([0, 5, 17, 64, 101, 191])
    rows = token_rows(hidden, logits, grad, cfg, bias, weights, tokens)
    assert torch.equal(rows.expert_indices, trace.expert_indices[tokens])
    _close(rows.out, out.detach()[tokens], fp32, "out rows")
    _close(rows.d_hidden, hr.grad[tokens], fp32, "d_hidden rows")
    _close(rows.d_logits, lr.grad[tokens], fp32, "d_logits rows")

    counts = trace.tokens_per_expert
    small = [int(e) for e in torch.argsort(counts)[:2]]
    Fd = w.ffn
    f_slice = (128, 256) if fp8 else (32, 64)
    res = expert_grads(hidden, logits, grad, cfg, bias, weights, small, f_slice=f_slice)
    c0, c1 = f_slice
    for e in small:
        if fp8:  # HF [out, in]: gate rows, then up rows
            full1 = torch.cat([g1.grad[e, c0:c1], g1.grad[e, Fd + c0:Fd + c1]])
            full2 = g2.grad[e, :, c0:c1]
        else:    # [H, 2F]: gate columns, then up columns
            full1 = torch.cat([g1.grad[e, :, c0:c1], g1.grad[e, :, Fd + c0:Fd + c1]], dim=1)
            full2 = g2.grad[e, c0:c1]
        _close(res.d_w1[e], full1, fp32, f"d_w1[{e}]")
        _close(res.d_w2[e], full2, fp32, f"d_w2[{e}]")


def _fp32_full_run():
    w = replace(C.QWEN3, tokens=192, hidden=128, ffn=96, experts=16, topk=4, dtype=torch.float32)
    hidden, logits, grad = C.make_hidden(w), C.make_logits(w), C.make_grad(w)
    bias = C.make_expert_bias(w)
    m1, m2 = C.make_weights(w)
    cfg = _cfg(w)
    w1r, w2r = m1.clone().requires_grad_(), m2.clone().requires_grad_()
    hr, lr = hidden.clone().requires_grad_(), logits.clone().requires_grad_()
    out, trace = o_layer.moe_layer(hr, lr, w1r, w2r, cfg, expert_bias=bias, trace=True)
    out.backward(grad)
    return w, (hidden, logits, grad, cfg, bias), (m1, m2), out.detach(), hr.grad, w1r.grad, trace


def _planted(m1, m2, mistake):
    """ExpertWeights whose ``select`` makes one slicing / renumbering mistake."""
    def getter(experts, f_slice):
        sel = ExpertWeights(w1=m1, w2=m2).select(experts, f_slice)
        if mistake == "swap_experts":  # renumbering: the first two selected experts trade weights
            order = torch.arange(experts.numel())
            order[[0, 1]] = order[[1, 0]]
            return ExpertWeights(w1=sel.w1[order].contiguous(), w2=sel.w2[order].contiguous())
        c0, c1 = f_slice  # up_from_gate: the up half of the slice is the gate's columns
        gate = m1[experts][:, :, c0:c1]
        return ExpertWeights(w1=torch.cat([gate, gate], dim=2).contiguous(), w2=sel.w2)

    return ExpertWeights(w1=m1, w2=m2, getter=getter)


@pytest.mark.parametrize("mistake", ["up_from_gate", "swap_experts"])
def test_sampled_oracle_planted_mistake_fails(mistake):
    """A slicing mistake (up columns taken from the gate half) or a renumbering
    mistake (two experts' weights swapped) in the sampled oracle makes its
    result differ from the full run well beyond the fp32 bound the GPU-side
    comparison relies on, so the decomposition check above would catch it."""
    w, inputs, (m1, m2), out, d_hidden, d_w1, trace = _fp32_full_run()
    hidden, logits, grad, cfg, bias = inputs
    bad = _planted(m1, m2, mistake)
    if mistake == "swap_experts":
        tokens = torch.arange(0, 192, 7)
        rows = token_rows(hidden, logits, grad, cfg, bias, bad, tokens)
        mx, _ = rel_errors(rows.out, out[tokens])
        assert mx > 1e-2, mx
        # the same call with the correct weights agrees
        good = token_rows(hidden, logits, grad, cfg, bias, ExpertWeights(w1=m1, w2=m2), tokens)
        assert rel_errors(good.out, out[tokens])[0] <= 1e-5
    else:
        counts = trace.tokens_per_expert
        e = int(torch.argsort(counts)[-1])
        c0, c1 = 32, 64
        Fd = w.ffn
        res = expert_grads(hidden, logits, grad, cfg, bias, bad, [e], f_slice=(c0, c1))
        full1 = torch.cat([d_w1[e, :, c0:c1], d_w1[e, :, Fd + c0:Fd + c1]], dim=1)
        mx, _ = rel_errors(res.d_w1[e], full1)
        assert mx > 1e-2, mx
        good = expert_grads(hidden, logits, grad, cfg, bias, ExpertWeights(w1=m1, w2=m2), [e],
                            f_slice=(c0, c1))
        assert rel_errors(good.d_w1[e], full1)[0] <= 1e-5
