"""Pin the CPU oracle to the reference's own known-answer tests (CPU).

Every literal below is taken from the reference test named in the comment;
the checks run the oracle's restatement (not the reference) on the same
inputs and compare with the same literal answers.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import fp8 as o_fp8
from oracle.native_providers import gated_activation as o_gated
from oracle.native_providers import grouped_matmul as o_gmm
from oracle.native_providers import moe_permutation as o_perm
from oracle.native_providers import routing as o_route
from torchturbo_amd.dispatch import MoEPermutation


# --- permutation / unpermutation ------------------------------------------------
def test_permutation_complete_result():
    # tests/ops/test_moe_permutation_contract.py:72-84
    rmap = torch.tensor([[False, True], [True, False]])
    r = o_perm.permute(torch.tensor([[2.0], [3.0]]), rmap,
                       probs=torch.tensor([[0.0, 0.5], [0.25, 0.0]]),
                       expert_indices=torch.tensor([[1], [0]]))
    assert r.tokens.tolist() == [[3.0], [2.0]]
    assert r.probs.tolist() == [0.25, 0.5]
    assert r.row_indices.tolist() == [[1], [0]] and r.row_indices.dtype == torch.int32


def test_mixed_provider_case_packed_rows_outputs_and_grads():
    # tests/ops/test_moe_permutation_contract.py:307-370 (torch/torch pairing)
    tokens = torch.tensor([[10.0], [20.0], [30.0]], requires_grad=True)
    probs = torch.tensor([[0.25, 0.0, 0.5], [0.0, 0.75, 0.125], [0.125, 0.25, 0.0]],
                         requires_grad=True)
    mask = probs.detach().bool()
    idx = torch.tensor([[0, 2], [1, 2], [0, 1]])
    m = o_perm.permute(tokens, mask, probs=probs, expert_indices=idx)
    assert m.tokens.detach().flatten().tolist() == [10.0, 30.0, 20.0, 30.0, 10.0, 20.0]
    assert m.row_indices.tolist() == [[0, 4], [2, 5], [1, 3]]
    g = torch.autograd.grad(m.probs.sum(), probs, retain_graph=True)[0]
    assert torch.equal(g, mask.float())
    out = o_perm.unpermute(m, tokens.shape, probs=probs)
    assert out.detach().flatten().tolist() == [7.5, 17.5, 11.25]
    out.sum().backward()
    torch.testing.assert_close(tokens.grad, probs.detach().sum(1, keepdim=True))
    torch.testing.assert_close(probs.grad, tokens.detach().expand_as(probs) * mask)
    assert o_perm.unpermute(m, tokens.shape).detach().flatten().tolist() == [20.0, 40.0, 60.0]


@pytest.mark.parametrize("dtype,large", [(torch.bfloat16, 256), (torch.float16, 2048)])
@pytest.mark.parametrize("weighted", [False, True])
def test_combine_keeps_small_contributions(dtype, large, weighted):
    # tests/ops/test_moe_permutation_contract.py:37-69: fp32 accumulation,
    # one rounding; slot order differs from expert order.
    packed = torch.tensor([[large], [-large], [1], [2], [-large], [large]], dtype=dtype,
                          requires_grad=True)
    probs = torch.full((2, 3), 0.5, requires_grad=True) if weighted else None
    perm = MoEPermutation(packed, None, torch.tensor([[0, 2, 4], [5, 1, 3]], dtype=torch.int32),
                          torch.tensor([[0, 1, 2], [2, 0, 1]]))
    out = o_perm.unpermute(perm, torch.Size([2, 1]), probs=probs)
    expected = torch.tensor([[1], [2]], dtype=dtype) * (0.5 if weighted else 1)
    torch.testing.assert_close(out, expected, rtol=0, atol=0)
    out.sum().backward()
    torch.testing.assert_close(packed.grad, torch.full_like(packed, 0.5 if weighted else 1))
    if weighted:
        torch.testing.assert_close(
            probs.grad, torch.tensor([[large, 1, -large], [-large, 2, large]]).float())


def test_unpermutation_keeps_probability_precision():
    # tests/ops/test_moe_permutation_contract.py:412-434
    packed = torch.tensor([[1.0], [-1.0]], dtype=torch.bfloat16, requires_grad=True)
    probs = torch.tensor([[1.00390625, 1.0]], requires_grad=True)
    m = MoEPermutation(packed, None, torch.tensor([[0, 1]], dtype=torch.int32),
                       torch.tensor([[0, 1]]))
    out = o_perm.unpermute(m, torch.Size([1, 1]), probs=probs)
    torch.testing.assert_close(out, torch.tensor([[0.00390625]], dtype=torch.bfloat16),
                               rtol=0, atol=0)
    out.sum().backward()
    torch.testing.assert_close(probs.grad, torch.tensor([[1.0, -1.0]]))


def test_zero_probability_selection_keeps_rows_and_router_grad():
    # tests/ops/test_moe_permutation_contract.py:228-247
    probs = torch.tensor([[0.0, 1.0]], requires_grad=True)
    r = o_perm.permute(torch.tensor([[2.0]]), torch.tensor([[True, True]]), probs=probs,
                       expert_indices=torch.tensor([[0, 1]]))
    assert r.tokens.tolist() == [[2.0], [2.0]] and r.probs.tolist() == [0.0, 1.0]
    (r.tokens * r.probs[:, None]).sum().backward()
    assert probs.grad.tolist() == [[2.0, 2.0]]


def test_sort_chunks():
    # tests/models/test_moe_permutation.py:101-151 form: chunks reordered by index
    x = torch.arange(10.0).view(10, 1)
    out, p = o_perm.sort_chunks(x, torch.tensor([3, 2, 5]), torch.tensor([2, 0, 1]),
                                probs=torch.arange(10.0))
    assert out.flatten().tolist() == [5, 6, 7, 8, 9, 0, 1, 2, 3, 4]
    assert p.tolist() == [5, 6, 7, 8, 9, 0, 1, 2, 3, 4]


# --- router ----------------------------------------------------------------------
@pytest.mark.parametrize("score", ["softmax", "sigmoid", "sqrtsoftplus"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_low_precision_scores_do_not_change_selected_expert(score, dtype):
    # tests/models/test_moe_router.py:74-83
    _, rmap, ids = o_route.topk_softmax_with_capacity(
        torch.tensor([[0.0, 0.0001]], dtype=dtype), 1, use_pre_softmax=True, score_function=score)
    assert rmap.tolist() == [[False, True]] and ids.tolist() == [[1]]


@pytest.mark.parametrize("score", ["sigmoid", "sqrtsoftplus"])
def test_probability_normalization_and_scaling_use_fp32(score):
    # tests/models/test_moe_router.py:86-111
    logits = torch.tensor([[2.0, 1.0, -1.0]], dtype=torch.bfloat16, requires_grad=True)
    ref = logits.detach().float().requires_grad_()
    fn = torch.sigmoid if score == "sigmoid" else (lambda x: F.softplus(x).sqrt())
    sel = fn(ref)[:, :2]
    expected = (sel / sel.sum(-1, keepdim=True) * 1.7).to(logits.dtype)
    probs, _, _ = o_route.topk_softmax_with_capacity(logits, 2, score_function=score,
                                                      scaling_factor=1.7)
    torch.testing.assert_close(probs[:, :2], expected, rtol=0, atol=0)
    g = torch.tensor([[1.0, 3.0]], dtype=logits.dtype)
    (probs[:, :2] * g).sum().backward()
    (expected * g).sum().backward()
    torch.testing.assert_close(logits.grad, ref.grad.to(logits.dtype), rtol=0, atol=0)


@pytest.mark.parametrize("pre", [False, True])
def test_softmax_normalization_precedes_scaling(pre):
    # tests/models/test_moe_router.py:150-171 (routing only)
    logits = torch.tensor([[2.0, 1.0, 0.0]], requires_grad=True)
    ref = logits.detach().clone().requires_grad_()
    expected = (ref.softmax(-1)[..., :2] if pre else ref[..., :2].softmax(-1)) * 2.0
    probs, _, _ = o_route.topk_softmax_with_capacity(logits, 2, use_pre_softmax=pre,
                                                      scaling_factor=2.0)
    torch.testing.assert_close(probs[:, :2], expected)
    (probs * torch.tensor([[1.0, 3.0, 0.0]])).sum().backward()
    (expected * torch.tensor([1.0, 3.0])).sum().backward()
    torch.testing.assert_close(logits.grad, ref.grad)


def test_group_limited_selection_kat():
    # tests/models/test_moe_adapter_routing.py:179-201: top-4 group sums favour
    # group 1 (2.4 > 1.72) although the two best single experts are in group 0.
    scores = torch.tensor([[0.9, 0.8, 0.01, 0.01, 0.6, 0.6, 0.6, 0.6]])
    probs, _, ids = o_route.topk_softmax_with_capacity(
        scores.logit(), 4, num_groups=2, group_topk=1, scaling_factor=1.0,
        score_function="sigmoid", expert_bias=torch.zeros(8))
    assert ids.sort(-1).values.tolist() == [[4, 5, 6, 7]]
    torch.testing.assert_close(probs, torch.tensor([[0., 0., 0., 0., .25, .25, .25, .25]]))


@pytest.mark.parametrize("score", ["softmax", "sigmoid", "sqrtsoftplus"])
@pytest.mark.parametrize("grouped", [False, True])
def test_topk_result_packs_weights_map_and_ids(score, grouped):
    # tests/models/test_moe_routing_result.py:11-49 (E=512, k=8, groups 8/4,
    # scale 2.5, bias): dense probs, map and ids describe the same selection.
    g = torch.Generator().manual_seed(71)
    logits = torch.randn(17, 512, generator=g, requires_grad=True)
    probs, rmap, ids = o_route.topk_softmax_with_capacity(
        logits, 8, use_pre_softmax=True, num_groups=8 if grouped else None,
        group_topk=4 if grouped else None, scaling_factor=2.5, score_function=score,
        expert_bias=torch.linspace(-0.01, 0.01, 512))
    assert probs.shape == rmap.shape == (17, 512)
    assert rmap.sum(-1).tolist() == [8] * 17
    order = ids.sort(-1).indices
    assert torch.equal(ids.gather(1, order), rmap.nonzero(as_tuple=True)[1].reshape(17, 8))
    torch.testing.assert_close(probs.gather(1, ids).gather(1, order),
                               probs.masked_select(rmap).reshape(17, 8), rtol=0, atol=0)


# --- grouped matmul ----------------------------------------------------------------
@pytest.mark.parametrize("trans_b", [False, True])
def test_grouped_matmul_forward_backward_form(trans_b):
    # tests/ops/npu/test_grouped_matmul.py:11-90: counts [0, 5, 0, 11],
    # grad_output of ones; explicit per-expert forward and backward.
    counts = [0, 5, 0, 11]
    g = torch.Generator().manual_seed(3)
    x = torch.randn(16, 6, generator=g, requires_grad=True)
    w = torch.randn(4, 7, 6, generator=g) if trans_b else torch.randn(4, 6, 7, generator=g)
    w.requires_grad_()
    y = o_gmm.grouped_matmul(x, w, counts, trans_b=trans_b)
    y.backward(torch.ones_like(y))
    gx = torch.zeros_like(x)
    gw = torch.zeros_like(w)
    start = 0
    for e, c in enumerate(counts):
        xs = x.detach()[start:start + c]
        go = torch.ones(c, 7)
        if trans_b:
            gx[start:start + c] = go @ w.detach()[e]
            gw[e] = (xs.T @ go).T
        else:
            gx[start:start + c] = go @ w.detach()[e].T
            gw[e] = xs.T @ go
        start += c
    torch.testing.assert_close(x.grad, gx)
    torch.testing.assert_close(w.grad, gw)
    assert torch.count_nonzero(w.grad[0]) == 0 and torch.count_nonzero(w.grad[2]) == 0


def test_grouped_matmul_rejects_bad_counts():
    with pytest.raises(ValueError, match="tokens_per_expert"):
        o_gmm.grouped_matmul(torch.ones(2, 3), torch.ones(2, 3, 4), [2])
    with pytest.raises(ValueError, match="shape"):
        o_gmm.grouped_matmul(torch.ones(2, 3), torch.ones(3, 4), [2])


# --- FP8 dequant --------------------------------------------------------------------
def test_apply_scales_kat():
    # tests/scripts/test_dequant.py:61-76: values [1, 2] times scales
    # [0.5, 2.0] give [0.5, 4.0] in bf16. With block scales the two values sit
    # in different 128-column blocks.
    w = torch.zeros(1, 129)
    w[0, 0], w[0, 128] = 1.0, 2.0
    out = o_fp8.dequantize_weight(w.to(torch.float8_e4m3fn), torch.tensor([[0.5, 2.0]]))
    assert out.dtype == torch.bfloat16 and out.is_contiguous()
    assert out[0, 0].item() == 0.5 and out[0, 128].item() == 4.0
    # :144-153 (FP8 1.0 with scale 2.0 -> 2.0)
    one = torch.tensor([[1.0]]).to(torch.float8_e4m3fn)
    assert o_fp8.dequantize_weight(one, torch.tensor([[2.0]])).float().item() == 2.0
    with pytest.raises(ValueError, match="does not match"):
        o_fp8.expand_block_scales(torch.ones(1, 1), 1, 200)


def test_partial_and_whole_blocks():
    # Block expansion of scripts/dequant/bailing.py:81-102: repeat 128 along
    # both dims, crop partial tail blocks; :229-238 (ones x 2.0 over 128x128).
    s = torch.tensor([[1.0, 2.0], [0.5, 0.25]])
    out = o_fp8.dequantize_weight(torch.ones(200, 150).to(torch.float8_e4m3fn), s)
    assert out.shape == (200, 150)
    assert out[0, 0].item() == 1.0 and out[0, 149].item() == 2.0
    assert out[199, 0].item() == 0.5 and out[199, 149].item() == 0.25
    assert out[127, 127].item() == 1.0 and out[128, 128].item() == 0.25
    out = o_fp8.dequantize_weight(torch.ones(128, 128).to(torch.float8_e4m3fn),
                                  torch.tensor([[2.0]]))
    assert torch.equal(out.float(), torch.full((128, 128), 2.0))


# --- gated activation ---------------------------------------------------------------
def test_gated_activation_limits():
    # native gated_activation semantics (ops/providers/native/gated_activation.py:15-44)
    x = torch.tensor([[3.0, -1.0, 5.0, -6.0]])  # gate [3, -1], up [5, -6]
    out = o_gated.gated_activation(x, activation_func=F.silu, limit=2.0)
    expect = F.silu(torch.tensor([2.0, -1.0])) * torch.tensor([2.0, -2.0])
    torch.testing.assert_close(out[0], expect)
    out = o_gated.gated_activation(x, activation_func=F.silu, limit=2.0,
                                   clamp_gate_after_activation=True)
    expect = F.silu(torch.tensor([3.0, -1.0])).clamp(max=2.0) * torch.tensor([2.0, -2.0])
    torch.testing.assert_close(out[0], expect)
    with pytest.raises(ValueError):
        o_gated.gated_activation(x, activation_func=torch.tanh)


def test_gated_activation_gelu_and_probs_closed_forms():
    # GELU gate: gelu(0) = 0 and gelu(x) -> x for large x (erf -> 1); the cap
    # before activation turns gelu(9) into gelu(2); probs scale each row.
    x = torch.tensor([[0.0, 9.0, 3.0, 1.5]], dtype=torch.float64)  # gate [0, 9], up [3, 1.5]
    out = o_gated.gated_activation(x, activation_func=F.gelu)
    assert out[0, 0].item() == 0.0
    assert abs(out[0, 1].item() - 9.0 * 1.5) < 1e-12
    capped = o_gated.gated_activation(x, activation_func=F.gelu, limit=2.0)
    expect = F.gelu(torch.tensor([0.0, 2.0], dtype=torch.float64)) * torch.tensor([2.0, 1.5],
                                                                                 dtype=torch.float64)
    torch.testing.assert_close(capped[0].double(), expect)
    p = torch.tensor([0.25], dtype=torch.float64)
    withp = o_gated.gated_activation_probs(x, p, activation_func=F.gelu, limit=2.0)
    torch.testing.assert_close(withp, capped * 0.25)


@pytest.mark.parametrize("fn", [F.silu, F.gelu])
@pytest.mark.parametrize("limit,after", [(0.0, False), (2.0, False), (2.0, True)])
def test_gated_activation_probs_gradcheck(fn, limit, after):
    # Gradients of the composition against finite differences. Without a cap
    # the math stays fp64 (strict check); with a cap the reference computes in
    # fp32 (``up.float()``), so the step and tolerance are sized for fp32, and
    # the points keep away from the cap (|x| and act(x) not within 0.05 of it).
    g = torch.Generator().manual_seed(3)
    x = torch.rand(5, 8, generator=g, dtype=torch.float64) * 6 - 3
    near = ((x.abs() - 2.0).abs() < 0.05) | ((fn(x) - 2.0).abs() < 0.05)
    x = torch.where(near, x + 0.2, x).requires_grad_()
    p = torch.rand(5, generator=g, dtype=torch.float64).requires_grad_()
    f = lambda a, b: o_gated.gated_activation_probs(  # noqa: E731
        a, b, activation_func=fn, limit=limit, clamp_gate_after_activation=after).double()
    if limit == 0:
        assert torch.autograd.gradcheck(f, (x, p))
    else:
        assert torch.autograd.gradcheck(f, (x, p), eps=1e-3, atol=2e-3, rtol=2e-3)
