"""The MoE layer on the GPU at the benchmark configurations' real sizes.

Qwen3-30B-A3B (16384 tokens), Mixtral (8192 x 4096 x 14336), DeepSeek-V3
(4096 tokens, 256 FP8 experts of 7168 x 2048 with 128x128 block scales, 56
scale blocks along the hidden size, plus the dense shared expert) and the
packed varlen batch (72,192 tokens, skewed routing with empty experts) run
forward and backward through the HIP providers at full size. The oracle
checks them where it can run in seconds (``tests/sampled_oracle.py``):

* routing of every token: the routing map and the per-expert counts are
  bit-exact (fp32 logits);
* output, d_hidden and d_logits rows of a seeded token sample;
* the weight gradients of the two least-loaded non-empty experts, of the
  most-loaded expert (the longest row-gathering reduction) and of one
  mid-loaded expert for the bf16 configurations, on an ffn column slice where
  the full width would not fit the oracle's budget; empty experts get exactly
  zero gradients.

Tolerance: normwise max relative error <= 2e-2, mean <= 2e-3 (bf16).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import layer as o_layer
from tests.conftest import assert_bf16_close
from tests.sampled_oracle import ExpertWeights, expert_grads, token_rows
from torchturbo_amd import configs as C
from torchturbo_amd.dispatch import OpPolicy
from torchturbo_amd.moe import Fp8GroupedMLP, GroupedMLP, MoEConfig, MoELayer, MoESubmodules, ModuleSpec
from torchturbo_amd.runtime import CudaRuntime

pytestmark = pytest.mark.gpu
DEV = "cuda"

# workload -> (sampled tokens for output rows, ffn slice for weight gradients or None,
#              also check one mid-loaded expert's gradient)
PLAN = {
    "qwen3_30b_a3b": (48, None, True),
    "mixtral": (16, (1024, 1280), True),
    "deepseek_v3": (6, (384, 512), False),
    "varlen_stress": (48, None, True),
}


def _routing_cfg(w):
    return o_layer.RoutingConfig(topk=w.topk, pre_softmax=w.pre_softmax,
                                 score_function=w.score_function, num_groups=w.num_groups,
                                 group_topk=w.group_topk, scaling_factor=w.scaling_factor)


def _gpu_layer(w):
    cfg = MoEConfig(
        hidden_size=w.hidden, num_moe_experts=w.experts, moe_ffn_hidden_size=w.ffn,
        gated_linear_unit=True, activation_func=F.silu, moe_router_topk=w.topk,
        moe_router_pre_softmax=w.pre_softmax, moe_router_score_function=w.score_function,
        moe_router_num_groups=w.num_groups, moe_router_group_topk=w.group_topk,
        moe_router_topk_scaling_factor=w.scaling_factor, params_dtype=w.dtype,
        moe_router_enable_expert_bias=w.expert_bias, perform_initialization=False,
    )
    experts = Fp8GroupedMLP if w.fp8 else GroupedMLP
    with torch.device(DEV):
        layer = MoELayer(cfg, None, submodules=MoESubmodules(experts=ModuleSpec(module=experts)))
    w1, w2 = C.make_weights(w, device=DEV)
    with torch.no_grad():
        if w.fp8:
            q1, s1 = C.fp8_blocks(w1.transpose(1, 2).contiguous())
            del w1
            q2, s2 = C.fp8_blocks(w2.transpose(1, 2).contiguous())
            del w2
            layer.experts.load_quantized(q1, s1, q2, s2)
            del q1, s1, q2, s2
            gpu_weights = ExpertWeights(q1=layer.experts.q1, s1=layer.experts.s1,
                                        q2=layer.experts.q2, s2=layer.experts.s2)

            def fetch(experts, f_slice):
                part = gpu_weights.select(experts.to(DEV), f_slice)
                return ExpertWeights(q1=part.q1.cpu(), s1=part.s1.cpu(), q2=part.q2.cpu(),
                                     s2=part.s2.cpu())
            cpu_weights = ExpertWeights(getter=fetch)
        else:
            layer.experts.weight1.copy_(w1.reshape(-1, 2 * w.ffn))
            layer.experts.weight2.copy_(w2.reshape(-1, w.hidden))
            cpu_weights = ExpertWeights(w1=w1.cpu(), w2=w2.cpu())
            del w1, w2
        bias = C.make_expert_bias(w)
        if bias is not None:
            layer.router.expert_bias.copy_(bias.to(DEV))
    shared_gpu = shared_cpu = None
    if w.shared_ffn:
        g = torch.Generator().manual_seed(w.seed + 9)
        mats = [(torch.randn(*s, generator=g) * 0.02).to(w.dtype)
                for s in ((w.shared_ffn, w.hidden), (w.shared_ffn, w.hidden),
                          (w.hidden, w.shared_ffn))]
        dev_mats = [m.to(DEV) for m in mats]

        def shared_gpu(x):
            return o_layer.dense_mlp(x, *dev_mats)

        def shared_cpu(x):
            return o_layer.dense_mlp(x, *mats)
    return layer, cpu_weights, bias, shared_gpu, shared_cpu


@pytest.mark.parametrize("name", list(PLAN))
def test_full_size_layer_matches_sampled_oracle(process_ops, name):
    process_ops(CudaRuntime(), OpPolicy.CUSTOM)
    w = C.resolve(C.WORKLOADS[name])
    n_rows, f_slice, mid_expert = PLAN[name]
    print(f"[full-size] {name}: T={w.tokens} H={w.hidden} E={w.experts} k={w.topk} F={w.ffn}",
          flush=True)
    hidden, logits, grad = C.make_hidden(w), C.make_logits(w), C.make_grad(w)
    cfg = _routing_cfg(w)
    layer, weights, bias, shared_gpu, shared_cpu = _gpu_layer(w)

    # GPU, full size
    hd = hidden.to(DEV).requires_grad_()
    ld = logits.to(DEV).requires_grad_()
    out = layer.forward_with_logits(hd, ld)
    if shared_gpu is not None:
        out = out + shared_gpu(hd)
    out.backward(grad.to(DEV))
    with torch.no_grad():
        _, rmap_d, ids_d = layer.router.routing(ld.detach())
    torch.cuda.synchronize()

    # routing of every token, bit-exact
    _, rmap_r, ids_r = o_layer.route(logits, cfg, bias)
    counts_r = rmap_r.sum(dim=0)
    assert torch.equal(rmap_d.cpu(), rmap_r)
    assert torch.equal(ids_d.cpu().sort(dim=1).values, ids_r.sort(dim=1).values)
    assert torch.equal(layer.token_dispatcher.tokens_per_expert.cpu(), counts_r)

    # sampled token rows
    g = torch.Generator().manual_seed(123)
    tokens = torch.randperm(w.tokens, generator=g)[:n_rows].sort().values
    rows = token_rows(hidden, logits, grad, cfg, bias, weights, tokens, shared=shared_cpu)
    assert_bf16_close(out.detach()[tokens.to(DEV)].cpu(), rows.out, what=f"{name} out rows")
    assert_bf16_close(hd.grad[tokens.to(DEV)].cpu(), rows.d_hidden, what=f"{name} d_hidden rows")
    assert_bf16_close(ld.grad[tokens.to(DEV)].cpu(), rows.d_logits, what=f"{name} d_logits rows")

    # weight gradients of the least-loaded non-empty experts, the most-loaded one
    # (the longest reduction: Qwen's top expert holds about 15.9k rows) and,
    # for the bf16 layers, one mid-loaded expert
    nonempty = (counts_r > 0).nonzero().flatten()
    order = nonempty[torch.argsort(counts_r[nonempty], stable=True)]
    chosen = [int(order[0]), int(order[1]), int(order[-1])]
    if mid_expert:
        chosen.append(int(order[len(order) // 2]))
    res = expert_grads(hidden, logits, grad, cfg, bias, weights, chosen, f_slice=f_slice,
                       full_ids=ids_r)
    Fd, H = w.ffn, w.hidden
    c0, c1 = f_slice if f_slice is not None else (0, Fd)
    for e in chosen:
        if w.fp8:  # master weights in HF [out, in] orientation
            g1 = layer.experts.master1.grad[e]
            g2 = layer.experts.master2.grad[e]
            got1 = torch.cat([g1[c0:c1], g1[Fd + c0:Fd + c1]])
            got2 = g2[:, c0:c1]
        else:
            g1 = layer.experts.weight1.grad.view(w.experts, H, 2 * Fd)[e]
            g2 = layer.experts.weight2.grad.view(w.experts, Fd, H)[e]
            got1 = torch.cat([g1[:, c0:c1], g1[:, Fd + c0:Fd + c1]], dim=1)
            got2 = g2[c0:c1]
        assert_bf16_close(got1.cpu(), res.d_w1[e], what=f"{name} d_w1[{e}] ({int(counts_r[e])} rows)")
        assert_bf16_close(got2.cpu(), res.d_w2[e], what=f"{name} d_w2[{e}] ({int(counts_r[e])} rows)")

    # empty experts: exactly zero weight gradients
    empty = (counts_r == 0).nonzero().flatten().tolist()
    if w.fp8:
        gw = (layer.experts.master1.grad, layer.experts.master2.grad)
    else:
        gw = (layer.experts.weight1.grad.view(w.experts, H, 2 * Fd),
              layer.experts.weight2.grad.view(w.experts, Fd, H))
    for e in empty:
        assert torch.count_nonzero(gw[0][e]) == 0 and torch.count_nonzero(gw[1][e]) == 0, e
    if name == "varlen_stress":
        assert len(empty) >= 8, "the varlen routing keeps 8 experts empty"
