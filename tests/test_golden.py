"""Committed golden vectors (``tests/golden/``) against the oracle (CPU) and
the HIP path (GPU).

Integer vectors (routing ids, packed-row maps, counts) must match exactly.
The toy layer (fp32) output / gradient slices match the oracle to 1e-5
relative (CPU kernels may sum in another order on another host) and the HIP
path to the fp32 tolerance of the layer test.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import layer as o_layer
from oracle import route_np
from oracle.native_providers import routing as o_route
from tests.conftest import rel_errors
from torchturbo_amd import configs as C

GOLDEN = Path(__file__).resolve().parent / "golden"


def cases():
    return json.loads((GOLDEN / "routing_cases.json").read_text())


def toy():
    return np.load(GOLDEN / "toy_layer.npz")


def test_oracle_reproduces_routing_cases():
    for c in cases():
        logits = torch.tensor(c["logits"], dtype=torch.float32)
        _, _, ids = o_route.topk_softmax_with_capacity(logits, c["k"])
        assert ids.tolist() == c["ids"]
        rows, tor, counts, _ = route_np.route_index(np.array(c["ids"]), c["E"])
        assert rows.tolist() == c["row_indices"]
        assert tor.tolist() == c["token_of_row"]
        assert counts.tolist() == c["counts"]


def _toy_oracle():
    w = C.TOY
    hidden, logits = C.make_hidden(w), C.make_logits(w)
    w1, w2 = C.make_weights(w)
    grad = C.make_grad(w)
    h = hidden.clone().requires_grad_()
    out, trace = o_layer.moe_layer(h, logits, w1, w2, o_layer.RoutingConfig(topk=w.topk),
                                   trace=True)
    out.backward(grad)
    return out.detach(), h.grad, trace


def test_oracle_reproduces_toy_layer():
    g = toy()
    out, dh, trace = _toy_oracle()
    assert np.array_equal(trace.expert_indices.numpy(), g["ids"])
    assert np.array_equal(trace.tokens_per_expert.numpy(), g["counts"])
    assert rel_errors(out[:64], torch.from_numpy(g["out_head"]))[0] <= 1e-5
    assert rel_errors(dh[:64], torch.from_numpy(g["dhidden_head"]))[0] <= 1e-5
    assert abs(out.norm().item() / g["norms"][0] - 1) <= 1e-5


@pytest.mark.gpu
def test_hip_routing_and_index_match_golden(hip_ops):
    from torchturbo_amd.providers.hip._functions import route_index

    for c in cases():
        logits = torch.tensor(c["logits"], dtype=torch.float32, device="cuda")
        _, rmap, ids = hip_ops.topk_softmax_with_capacity(logits, c["k"])
        assert ids.cpu().tolist() == c["ids"]
        rows, tor, _, counts = route_index(ids, c["E"], None)
        assert rows.cpu().tolist() == c["row_indices"]
        assert tor.cpu().tolist() == c["token_of_row"]
        assert counts.cpu().tolist() == c["counts"]


@pytest.mark.gpu
def test_hip_toy_layer_matches_golden(process_ops):
    import torch.nn.functional as F

    from torchturbo_amd.dispatch import OpPolicy
    from torchturbo_amd.moe import GroupedMLP, MoEConfig, MoELayer, MoESubmodules, ModuleSpec
    from torchturbo_amd.runtime import CudaRuntime

    process_ops(CudaRuntime(), OpPolicy.CUSTOM)
    g = toy()
    w = C.TOY
    hidden, logits = C.make_hidden(w), C.make_logits(w)
    w1, w2 = C.make_weights(w)
    grad = C.make_grad(w)
    cfg = MoEConfig(hidden_size=w.hidden, num_moe_experts=w.experts, moe_ffn_hidden_size=w.ffn,
                    gated_linear_unit=True, activation_func=F.silu, moe_router_topk=w.topk)
    layer = MoELayer(cfg, None, submodules=MoESubmodules(experts=ModuleSpec(module=GroupedMLP)))
    layer = layer.cuda()
    with torch.no_grad():
        layer.experts.weight1.copy_(w1.reshape(-1, 2 * w.ffn))
        layer.experts.weight2.copy_(w2.reshape(-1, w.hidden))
    h = hidden.cuda().requires_grad_()
    out = layer.forward_with_logits(h, logits.cuda())
    out.backward(grad.cuda())
    assert np.array_equal(layer.token_dispatcher.tokens_per_expert.cpu().numpy(), g["counts"])
    assert rel_errors(out.detach()[:64].cpu(), torch.from_numpy(g["out_head"]))[0] <= 1e-4
    assert rel_errors(h.grad[:64].cpu(), torch.from_numpy(g["dhidden_head"]))[0] <= 1e-4
