"""Host-side composition: the product MoELayer on the CPU with the oracle's
native providers attached, against the oracle layer and the dense loop.

These check the host logic (router -> dispatcher stages -> experts ->
combine, shapes, dtypes, gradients) without a GPU; the HIP kernels
themselves are checked in the ``gpu`` tests.
"""

from __future__ import annotations

from dataclasses import replace

import pytest
import torch
import torch.nn.functional as F

from oracle import dense as o_dense
from oracle import layer as o_layer
from torchturbo_amd import configs as C
from torchturbo_amd.dispatch import OpPolicy
from torchturbo_amd.moe import GroupedMLP, MoEConfig, MoELayer, MoESubmodules, ModuleSpec
from torchturbo_amd.runtime import CpuRuntime


def make_layer(w, w1, w2):
    cfg = MoEConfig(hidden_size=w.hidden, num_moe_experts=w.experts, moe_ffn_hidden_size=w.ffn,
                    gated_linear_unit=True, activation_func=F.silu, moe_router_topk=w.topk,
                    moe_router_pre_softmax=w.pre_softmax, params_dtype=w.dtype)
    layer = MoELayer(cfg, None, submodules=MoESubmodules(experts=ModuleSpec(module=GroupedMLP)))
    with torch.no_grad():
        layer.experts.weight1.copy_(w1.reshape(-1, 2 * w.ffn))
        layer.experts.weight2.copy_(w2.reshape(-1, w.hidden))
    return layer


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_product_layer_on_cpu_matches_oracle_layer(process_ops, dtype):
    process_ops(CpuRuntime(), OpPolicy.NATIVE, oracle=True)
    w = replace(C.TOY, tokens=64, hidden=32, ffn=16, experts=8, dtype=dtype)
    hidden, logits = C.make_hidden(w), C.make_logits(w)
    w1, w2 = C.make_weights(w)
    grad = C.make_grad(w)
    layer = make_layer(w, w1, w2)
    h = hidden.clone().requires_grad_()
    lg = logits.clone().requires_grad_()
    out = layer.forward_with_logits(h, lg)
    out.backward(grad)
    hr = hidden.clone().requires_grad_()
    lr = logits.clone().requires_grad_()
    w1r, w2r = w1.clone().requires_grad_(), w2.clone().requires_grad_()
    ref = o_layer.moe_layer(hr, lr, w1r, w2r, o_layer.RoutingConfig(topk=w.topk))
    ref.backward(grad)
    # Same native ops in the same order: bit-identical.
    assert torch.equal(out, ref)
    assert torch.equal(h.grad, hr.grad)
    assert torch.equal(lg.grad, lr.grad)
    assert torch.equal(layer.experts.weight1.grad.view_as(w1r.grad), w1r.grad)
    assert torch.equal(layer.experts.weight2.grad.view_as(w2r.grad), w2r.grad)


def test_oracle_layer_matches_dense_loop():
    w = replace(C.TOY, tokens=48, hidden=16, ffn=8, experts=6, topk=2)
    hidden, logits = C.make_hidden(w), C.make_logits(w)
    w1, w2 = C.make_weights(w)
    out, trace = o_layer.moe_layer(hidden, logits, w1, w2, o_layer.RoutingConfig(topk=2), trace=True)
    topk_probs = trace.probs.gather(1, trace.expert_indices)
    dense = o_dense.dense_moe(hidden, trace.expert_indices, topk_probs, w1, w2)
    torch.testing.assert_close(out, dense, rtol=1e-5, atol=1e-6)


def test_layer_forward_computes_logits_with_gating(process_ops):
    process_ops(CpuRuntime(), OpPolicy.NATIVE, oracle=True)
    w = replace(C.TOY, tokens=10, hidden=8, ffn=4, experts=4, topk=2)
    torch.manual_seed(0)
    cfg = MoEConfig(hidden_size=w.hidden, num_moe_experts=w.experts, moe_ffn_hidden_size=w.ffn,
                    gated_linear_unit=True, activation_func=F.silu, moe_router_topk=w.topk)
    layer = MoELayer(cfg, None, submodules=MoESubmodules(experts=ModuleSpec(module=GroupedMLP)))
    with torch.no_grad():
        for p in layer.parameters():
            p.normal_(std=0.3)
    x = torch.randn(2, 5, w.hidden, requires_grad=True)
    out, logits = layer(x)
    assert out.shape == x.shape and logits.shape == (10, 4)
    out.sum().backward()
    assert layer.router.weight.grad is not None and torch.count_nonzero(layer.router.weight.grad) > 0


def test_softmax_layer_preserves_router_probabilities_and_gradients(process_ops):
    # tests/models/test_moe_probability_weighting.py:100-131, restated
    process_ops(CpuRuntime(), OpPolicy.NATIVE, oracle=True)
    for topk, pre, scale in ((1, True, None), (1, True, 2.0), (2, True, 2.0), (2, False, 2.0)):
        cfg = MoEConfig(hidden_size=1, moe_ffn_hidden_size=1, num_moe_experts=3,
                        activation_func=torch.nn.Identity(), moe_router_topk=topk,
                        moe_router_pre_softmax=pre, moe_router_topk_scaling_factor=scale)
        layer = MoELayer(cfg, None, submodules=MoESubmodules(experts=ModuleSpec(module=GroupedMLP)))
        with torch.no_grad():
            layer.router.weight.copy_(torch.tensor([[2.0], [1.0], [0.0]]))
            layer.experts.weight1.fill_(1.0)
            layer.experts.weight2.copy_(torch.tensor([[1.0], [2.0], [3.0]]))
        ref_logits = layer.router.weight.detach().flatten().requires_grad_()
        ref_probs = ref_logits.softmax(-1)[:topk] if pre else ref_logits[:topk].softmax(-1)
        expected = (ref_probs * torch.arange(1, topk + 1)).sum()
        if scale is not None:
            expected = expected * scale
        out, _ = layer(torch.ones(1, 1, 1))
        torch.testing.assert_close(out.squeeze(), expected)
        out.sum().backward()
        expected.backward()
        torch.testing.assert_close(layer.router.weight.grad.flatten(), ref_logits.grad)


def test_folded_permutation_shape_rule():
    """Where the layer folds the permutation into the GEMMs (shape rule only; the
    GPU tests check the results): Qwen3-30B-A3B and the varlen batch yes, Mixtral's
    wide experts, small batches, fp32 and odd hidden sizes no."""
    from torchturbo_amd.providers.hip.fused_experts import shapes_pay

    bf = torch.bfloat16
    assert shapes_pay(16384, 2048, 1536, 8, 128, bf)            # Qwen3-30B-A3B
    assert shapes_pay(72192, 2048, 1536, 8, 128, bf)            # varlen stress
    assert not shapes_pay(8192, 4096, 28672, 2, 8, bf)          # Mixtral: fc1 7x hidden
    assert not shapes_pay(4096, 2048, 1536, 8, 128, bf)         # 256 rows per expert
    assert not shapes_pay(16384, 2048, 1536, 8, 128, torch.float32)
    assert not shapes_pay(16384, 2000, 1536, 8, 128, bf)        # hidden not a multiple of 64
    assert not shapes_pay(16384, 64, 128, 8, 16, bf)            # hidden of one k-tile
    # more experts than the gathering kernels' LDS schedule holds (about 636):
    # the layer keeps the permutation instead of failing in forward
    assert shapes_pay(40000, 2048, 1536, 8, 600, bf)
    assert not shapes_pay(131072, 2048, 1536, 8, 1024, bf)
