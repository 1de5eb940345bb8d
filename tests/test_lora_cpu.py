"""Grouped expert LoRA (``GroupedMLPLoRA``) on the CPU with the oracle's native
providers: the per-expert loop of ``tests/engine/test_grouped_mlp_lora.py:18-108``
(bit-exact with the same native ops), zero-token ranks, merge / unmerge, legacy
2-D checkpoints and argument errors (``src/torchturbo/engine/peft/lora.py``)."""

from __future__ import annotations

import copy

import pytest
import torch
import torch.nn.functional as F

from torchturbo_amd.dispatch import OpPolicy
from torchturbo_amd.moe import GroupedMLP, GroupedMLPLoRA, MoEConfig
from torchturbo_amd.runtime import CpuRuntime


def small_base(dtype=torch.bfloat16, experts=2):
    cfg = MoEConfig(hidden_size=4, moe_ffn_hidden_size=3, gated_linear_unit=True,
                    activation_func=F.silu, params_dtype=dtype)
    return GroupedMLP(num_local_experts=experts, use_te=False, config=cfg)


@pytest.mark.parametrize("use_lora", [False, True])
@pytest.mark.parametrize("num_tokens", [0, 3])
def test_experts_with_lora_match_per_expert_loop(process_ops, use_lora, num_tokens):
    process_ops(CpuRuntime(), OpPolicy.NATIVE, oracle=True)
    torch.manual_seed(13)
    base = small_base()
    if use_lora:
        base.requires_grad_(False)
    cand = GroupedMLPLoRA(base, "default", r=2, lora_alpha=4) if use_lora else base
    with torch.no_grad():
        for p in cand.parameters():
            p.normal_(std=.2)
    ref = copy.deepcopy(cand)
    x = torch.randn(num_tokens, 4, dtype=torch.bfloat16, requires_grad=True)
    rx = x.detach().clone().requires_grad_()
    probs = torch.tensor([.5005, .1237, .9953])[:num_tokens].requires_grad_()
    rprobs = probs.detach().clone().requires_grad_()
    counts = torch.tensor([2, 1] if num_tokens else [0, 0])
    got, _ = cand(x, counts, probs)

    rbase = ref.base_layer if use_lora else ref
    w1 = rbase.weight1.view(2, 4, 6)
    w2 = rbase.weight2.view(2, 3, 4)
    outs = []
    for e, (tok, p) in enumerate(zip(rx.split(counts.tolist()), rprobs.split(counts.tolist()))):
        h = tok @ w1[e]
        if use_lora:
            d = tok.float() @ ref.lora_A["default"].weight[e] @ ref.lora_B["default"].weight[e]
            h = h + d.to(h.dtype) * ref.scaling["default"]
        gate, up = h.chunk(2, dim=-1)
        a = ((F.silu(gate) * up) * p[:, None]).to(h.dtype)
        o = a @ w2[e]
        if use_lora:
            d = a.float() @ ref.lora_A2["default"].weight[e] @ ref.lora_B2["default"].weight[e]
            o = o + d.to(o.dtype) * ref.scaling["default"]
        outs.append(o)
    expect = torch.cat(outs)
    torch.testing.assert_close(got, expect, rtol=0, atol=0)
    g = torch.randn_like(got)
    got.backward(g)
    expect.backward(g)
    torch.testing.assert_close(x.grad, rx.grad)
    torch.testing.assert_close(probs.grad, rprobs.grad)
    for p, rp in zip(cand.parameters(), ref.parameters(), strict=True):
        torch.testing.assert_close(p.grad, rp.grad)


@pytest.mark.parametrize("experts", [1, 2])
def test_zero_token_forward_keeps_adapters_in_graph(process_ops, experts):
    process_ops(CpuRuntime(), OpPolicy.NATIVE, oracle=True)
    torch.manual_seed(0)
    lora = GroupedMLPLoRA(small_base(torch.float32, experts), "default", r=2, lora_alpha=4)
    h = torch.empty(0, 4, requires_grad=True)
    out, _ = lora(h, torch.zeros(experts, dtype=torch.long), torch.empty(0))
    out.sum().backward()
    assert out.shape == (0, 4)
    adapters = {n: p for n, p in lora.named_parameters() if n.startswith("lora_")}
    assert len(adapters) == 4
    for name, p in adapters.items():
        assert p.grad is not None and not p.grad.any(), name


def test_merge_unmerge_round_trip(process_ops):
    process_ops(CpuRuntime(), OpPolicy.NATIVE, oracle=True)
    torch.manual_seed(1)
    base = small_base(torch.float64)
    with torch.no_grad():
        base.weight1.normal_(std=.3)
        base.weight2.normal_(std=.3)
    lora = GroupedMLPLoRA(base, "default", r=2, lora_alpha=3, init_lora_weights="gaussian")
    with torch.no_grad():
        for p in (lora.lora_B["default"].weight, lora.lora_B2["default"].weight):
            p.normal_(std=.2)
        for n, p in lora.named_parameters():
            if n.startswith("lora_"):
                p.data = p.data.double()
    x = torch.randn(5, 4, dtype=torch.float64)
    counts, probs = torch.tensor([3, 2]), torch.rand(5, dtype=torch.float64)
    w1, w2 = base.weight1.detach().clone(), base.weight2.detach().clone()
    unmerged, _ = lora(x, counts, probs)
    lora.merge()
    assert lora.merged_adapters == ["default"]
    merged, _ = lora(x, counts, probs)
    torch.testing.assert_close(merged, unmerged, rtol=1e-12, atol=1e-12)
    lora.unmerge()
    torch.testing.assert_close(base.weight1, w1, rtol=0, atol=1e-14)
    torch.testing.assert_close(base.weight2, w2, rtol=0, atol=1e-14)
    lora.enable_adapters(False)
    plain, _ = lora(x, counts, probs)
    ref, _ = base(x, counts, probs)
    torch.testing.assert_close(plain, ref, rtol=0, atol=0)


def test_legacy_2d_checkpoint_converts_to_3d():
    torch.manual_seed(2)
    E, r = 2, 3
    lora = GroupedMLPLoRA(small_base(torch.float32, E), "default", r=r, lora_alpha=4)
    want = {k: torch.randn_like(v) for k, v in lora.state_dict().items() if k.startswith("lora_")}
    legacy = {}
    for k, v in want.items():
        if ".lora_A" in "." + k or k.startswith("lora_A"):
            legacy[k] = v.permute(0, 2, 1).reshape(E * r, -1)      # [r*E, in], expert-major rows
        else:
            legacy[k] = v.reshape(E * r, -1).T.contiguous()         # [out, r*E]
    state = dict(lora.state_dict())
    state.update(legacy)
    lora.load_state_dict(state)
    for k, v in want.items():
        torch.testing.assert_close(lora.state_dict()[k], v, rtol=0, atol=0)
    # the stated layout of B: new[e, k, o] = old[o, e*r + k]
    old_b = legacy["lora_B.default.weight"]
    assert torch.equal(lora.lora_B["default"].weight[1, 2], old_b[:, 1 * r + 2])


def test_lora_argument_errors():
    base = small_base(torch.float32)
    with pytest.raises(ValueError, match="DoRA"):
        GroupedMLPLoRA(base, "default", r=2, use_dora=True)
    with pytest.raises(ValueError, match="lora_bias"):
        GroupedMLPLoRA(base, "default", r=2, lora_bias=True)
    with pytest.raises(ValueError, match="positive integer"):
        GroupedMLPLoRA(base, "default", r=0)
    lora = GroupedMLPLoRA(base, "default", r=2, lora_alpha=8, use_rslora=True)
    assert lora.scaling["default"] == pytest.approx(8 / 2 ** 0.5)
    with pytest.raises(ValueError, match="not found"):
        lora.set_adapter("other")
