"""Router aux (load-balancing) loss and z-loss on the CPU oracle.

Closed forms of the reference's router tests, restated (not their code):
``tests/models/test_moe_router.py:137-243`` (empty source rank; hash and
learned layers with main, z and aux gradients) and
``tests/models/deepseek_v4/test_mtp_router_padding.py:196-220`` (padding rows
excluded from both losses and their metrics). ``router_loss_stats`` of the
oracle is pinned against brute force on tiny inputs.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle.native_providers.routing import router_loss_stats
from tests.conftest import assert_bf16_close
from torchturbo_amd.dispatch import OpPolicy
from torchturbo_amd.moe import MoEConfig, TopKRouter
from torchturbo_amd.moe.router import MoEAuxLossAutoScaler
from torchturbo_amd.runtime import CpuRuntime


@pytest.fixture
def cpu_ops(process_ops, monkeypatch):
    monkeypatch.setattr(MoEAuxLossAutoScaler, "loss_scale", 1.0)
    process_ops(CpuRuntime(), OpPolicy.NATIVE, oracle=True)


def test_z_loss_is_zero_for_an_empty_source_rank(cpu_ops):
    router = TopKRouter(MoEConfig(hidden_size=2, num_moe_experts=4, moe_router_topk=2,
                                  moe_z_loss_coeff=0.3))
    inputs = torch.empty(0, 1, 2, requires_grad=True)
    probs, _, _, _ = router(inputs)
    metrics = router.pop_metrics()
    torch.testing.assert_close(metrics["z_loss"], torch.tensor(0.0))
    torch.testing.assert_close(metrics["z_loss_scaled"], torch.tensor(0.0))
    probs.sum().backward()
    torch.testing.assert_close(router.weight.grad, torch.zeros_like(router.weight))


@pytest.mark.parametrize("score_function", ["softmax", "sigmoid", "sqrtsoftplus"])
@pytest.mark.parametrize("layer_number", [0, 1], ids=["hash", "learned"])
@pytest.mark.parametrize("z_coeff", [0.0, 0.3])
def test_main_z_and_aux_gradients_match_closed_form(cpu_ops, score_function, layer_number,
                                                    z_coeff):
    router = TopKRouter(
        MoEConfig(hidden_size=2, num_moe_experts=4, moe_router_topk=2,
                  moe_router_score_function=score_function, moe_router_pre_softmax=True,
                  num_hash_layers=1, vocab_size=2, moe_aux_loss_coeff=0.2,
                  moe_z_loss_coeff=z_coeff),
        layer_number=layer_number,
    )
    table = torch.tensor([[0, 1], [2, 3]])
    with torch.no_grad():
        router.weight.copy_(torch.tensor([[0.5, 0.1], [0.2, -0.3], [-0.4, 0.7], [0.6, -0.5]]))
        if layer_number == 0:
            router.tid2eid.copy_(table)
    x = torch.tensor([[[1.0, 2.0], [2.0, -1.0]]], requires_grad=True)
    rx = x.detach().clone().requires_grad_()
    rw = router.weight.detach().clone().requires_grad_()
    logits = F.linear(rx, rw).reshape(-1, 4)
    scores = {"softmax": logits.softmax(-1), "sigmoid": logits.sigmoid(),
              "sqrtsoftplus": F.softplus(logits).sqrt()}[score_function]
    idx = table if layer_number == 0 else scores.topk(2, dim=-1).indices
    sel = scores.gather(1, idx)
    if score_function != "softmax":
        sel = sel / sel.sum(-1, keepdim=True)
    want_probs = torch.zeros_like(scores).scatter(1, idx, sel)
    c = torch.tensor([[1.0, 2.0, 4.0, 8.0], [3.0, 5.0, 2.0, 1.0]])
    loss = (want_probs * c).sum() + z_coeff * logits.logsumexp(-1).square().mean()
    if layer_number == 1:
        # aux = E * sum_e(sum_t s_te * n_e) / (k * N^2), s normalised over experts
        n = torch.bincount(idx.flatten(), minlength=4)
        s = scores / scores.sum(-1, keepdim=True)
        loss = loss + 0.2 * 4 * (s.sum(0) * n).sum() / (2 * 2 ** 2)
    probs, rmap, _, _ = router(x, input_ids=torch.tensor([[0, 1]]))
    (probs * c).sum().backward()
    loss.backward()
    torch.testing.assert_close(probs, want_probs)
    torch.testing.assert_close(rmap, want_probs != 0)
    torch.testing.assert_close(router.weight.grad, rw.grad)
    torch.testing.assert_close(x.grad, rx.grad)
    metrics = router.pop_metrics()
    assert ("aux_loss" in metrics) == (layer_number == 1)
    assert ("z_loss" in metrics) == (z_coeff > 0)


@pytest.mark.parametrize("valid_rows", [[1, 0, 1, 1, 0], [0, 0, 0, 0, 0], [1, 1, 1, 1, 1]])
def test_padding_rows_leave_both_losses(cpu_ops, valid_rows):
    torch.manual_seed(3)
    E, k = 3, 2
    router = TopKRouter(MoEConfig(hidden_size=4, num_moe_experts=E, moe_router_topk=k,
                                  moe_router_score_function="sigmoid", moe_router_dtype="fp32",
                                  moe_aux_loss_coeff=0.05, moe_z_loss_coeff=0.02))
    valid = torch.tensor(valid_rows, dtype=torch.bool)
    logits = torch.randn(valid.numel(), E, requires_grad=True)
    ref = logits.detach().clone().requires_grad_()
    probs, _, _ = router.routing(logits, padding_mask=~valid)
    (probs * 0).sum().backward()  # only the two losses reach the logits
    lv = ref[valid]
    if lv.size(0):
        s = lv.sigmoid()
        n = torch.bincount(s.topk(k, dim=-1).indices.flatten(), minlength=E)
        s = s / s.sum(-1, keepdim=True)
        aux = E * (s.sum(0) * n).sum() / (k * lv.size(0) ** 2)
        z = lv.logsumexp(-1).square().mean()
    else:
        aux = z = ref.sum() * 0
    (0.05 * aux + 0.02 * z).backward()
    torch.testing.assert_close(logits.grad, ref.grad)
    assert not logits.grad[~valid].any()
    m = router.pop_metrics()
    torch.testing.assert_close(m["aux_loss_scaled"], aux.detach() * 0.05)
    torch.testing.assert_close(m["z_loss_scaled"], z.detach() * 0.02)


@pytest.mark.parametrize("score_function", ["softmax", "sigmoid", "sqrtsoftplus"])
def test_oracle_loss_stats_against_brute_force(score_function):
    """Per-row loops: scores by their definition, the top-k set as the k
    largest by a full sort (ties: lower id), log-sum-exp by math.log/exp."""
    import math

    g = torch.Generator().manual_seed(11)
    T, E, k = 6, 5, 2
    logits = torch.randn(T, E, generator=g, dtype=torch.float64).float()
    pad = torch.tensor([0, 1, 0, 0, 1, 0], dtype=torch.bool)
    ps, cn, zs = router_loss_stats(logits, k, score_function, pad)
    want_p = [0.0] * E
    want_c = [0] * E
    want_z = 0.0
    for t in range(T):
        if pad[t]:
            continue
        row = [float(v) for v in logits[t]]
        if score_function == "softmax":
            m = max(row)
            ex = [math.exp(v - m) for v in row]
            s = [v / sum(ex) for v in ex]
        else:
            f = ((lambda v: 1 / (1 + math.exp(-v))) if score_function == "sigmoid"
                 else (lambda v: math.sqrt(math.log1p(math.exp(v)))))
            r = [f(v) for v in row]
            s = [v / (sum(r) + 1e-20) for v in r]
        for e in range(E):
            want_p[e] += s[e]
        for e in sorted(range(E), key=lambda e: (-s[e], e))[:k]:
            want_c[e] += 1
        m = max(row)
        want_z += (m + math.log(sum(math.exp(v - m) for v in row))) ** 2
    torch.testing.assert_close(ps.double(), torch.tensor(want_p, dtype=torch.float64),
                               rtol=1e-5, atol=1e-6)
    assert cn.tolist() == want_c
    torch.testing.assert_close(zs.double(), torch.tensor(want_z, dtype=torch.float64),
                               rtol=1e-5, atol=1e-6)


def test_oracle_loss_stats_switches_and_padding_invariants():
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(7, 4, generator=g)
    ps, cn, zs = router_loss_stats(logits, 3, "softmax", aux=False, z=False)
    assert not ps.any() and not cn.any() and zs == 0
    ps, cn, zs = router_loss_stats(logits, 3, "softmax")
    # softmax rows sum to one; every valid token is counted k times
    torch.testing.assert_close(ps.sum(), torch.tensor(7.0))
    assert int(cn.sum()) == 7 * 3
    # padding every row leaves zeros; padding none equals no mask
    full = torch.ones(7, dtype=torch.bool)
    p0, c0, z0 = router_loss_stats(logits, 3, "softmax", full)
    assert not p0.any() and not c0.any() and z0 == 0
    for a, b in zip(router_loss_stats(logits, 3, "softmax", ~full), (ps, cn, zs)):
        torch.testing.assert_close(a, b)
    # a row's contribution does not depend on the other rows
    parts = [router_loss_stats(logits[i:i + 1], 3, "softmax") for i in range(7)]
    for j, whole in enumerate((ps, cn, zs)):
        torch.testing.assert_close(sum(p[j] for p in parts), whole)


@pytest.mark.parametrize("rdt", [None, "fp32"])
def test_fused_gate_path_equals_reference_composition(cpu_ops, rdt):
    """bf16 router weight, E a multiple of 32: forward takes the fused
    gating + top-k op; its outputs, losses and gradients equal the reference
    composition (gating, then routing) run on the same module."""
    torch.manual_seed(6)
    cfg = MoEConfig(hidden_size=64, num_moe_experts=64, moe_router_topk=4,
                    moe_router_dtype=rdt, moe_aux_loss_coeff=0.01, moe_z_loss_coeff=0.002,
                    params_dtype=torch.bfloat16)
    router = TopKRouter(cfg)
    torch.nn.init.normal_(router.weight, std=0.1)
    x = torch.randn(3, 5, 64).bfloat16()
    assert router._can_fuse_gate(x)
    w = torch.randn(15, 64)

    def run(fused):
        router.weight.grad = None
        xi = x.clone().requires_grad_()
        if fused:
            probs, rmap, ids, logits = router(xi)
        else:
            logits = router.gating(xi)
            probs, rmap, ids = router.routing(logits)
        ((probs.float() * w).sum() + logits.float().square().sum() * 1e-3).backward()
        return probs, rmap, ids, logits, xi.grad, router.weight.grad.clone(), router.pop_metrics()

    a, b = run(True), run(False)
    for u, v in zip(a[:4], b[:4]):  # probs, map, ids, logits: the same ops
        assert torch.equal(u, v)
    for key in ("aux_loss", "z_loss"):
        torch.testing.assert_close(a[6][key], b[6][key], rtol=0, atol=0)
    # autograd adds the logits' gradient terms in another order: in a bf16
    # router dtype that moves the last bit of some sums
    for u, v in zip(a[4:6], b[4:6]):
        if rdt is None:
            assert_bf16_close(u, v)
        else:
            torch.testing.assert_close(u, v)


def test_oracle_loss_stats_match_golden_brute_force():
    """tests/golden/router_loss_cases.json: per-row brute force in Python floats
    (make_golden.py), padding rows included."""
    import json
    import os

    path = os.path.join(os.path.dirname(__file__), "golden", "router_loss_cases.json")
    with open(path) as f:
        cases = json.load(f)
    for c in cases:
        logits = torch.tensor(c["logits"], dtype=torch.float32)
        pad = torch.tensor(c["padding_mask"], dtype=torch.bool)
        ps, cn, zs = router_loss_stats(logits, c["k"], c["score_function"], pad)
        torch.testing.assert_close(ps.double(), torch.tensor(c["prob_sum"], dtype=torch.float64),
                                   rtol=1e-5, atol=1e-6)
        assert cn.tolist() == c["tokens_per_expert"]
        torch.testing.assert_close(zs.double(), torch.tensor(c["z_sum"], dtype=torch.float64),
                                   rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("kwargs,match", [
    (dict(num_moe_experts=2048, moe_router_topk=8), "num_moe_experts=2048"),
    (dict(num_moe_experts=128, moe_router_topk=65), "moe_router_topk=65"),
])
def test_router_refuses_what_the_kernels_cannot_route_at_build(kwargs, match):
    """A router the HIP kernels cannot serve (more than 1024 experts, k above 64)
    raises when the layer is built, not on its first call."""
    with pytest.raises(ValueError, match=match):
        TopKRouter(MoEConfig(hidden_size=8, **kwargs))
    TopKRouter(MoEConfig(hidden_size=8, num_moe_experts=1024, moe_router_topk=64))
    TopKRouter(MoEConfig(hidden_size=8, num_moe_experts=64, moe_router_topk=4,
                         moe_router_dtype="fp64"))
