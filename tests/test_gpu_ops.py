"""HIP kernels vs the CPU oracle, op by op (GPU).

Integer results (routing ids, routing map, packed-row map, counts, packed
rows) are compared bit-exactly. The fp32-accumulated gather-sums are
compared bit-exactly too (same order, same rounding as the reference's CPU
``scatter_add_`` / ``index_add_``). Floating-point math that goes through
``exp`` or a GEMM is compared within the path's tolerance: normwise max
relative error <= 2e-2 and mean relative error <= 2e-3 for bf16 (tighter
for fp32 where stated).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.native_providers import grouped_matmul as o_gmm
from oracle.native_providers import moe_permutation as o_perm
from oracle.native_providers import routing as o_route
from oracle.native_providers import swiglu as o_swiglu
from oracle import fp8 as o_fp8
from oracle.native_providers import gated_activation as o_gated
from oracle import route_np
from tests.conftest import assert_bf16_close, rel_errors
from torchturbo_amd.dispatch import MoEPermutation, OpPolicy

pytestmark = pytest.mark.gpu
DEV = "cuda"


def distinct_ids(T, E, k, seed, skew=False):
    g = torch.Generator().manual_seed(seed)
    scores = torch.rand(T, E, generator=g)
    if skew:
        scores += torch.linspace(2.0, 0.0, E)
    return scores.topk(k, dim=1).indices


# ---------------------------------------------------------------------------
# Router
# ---------------------------------------------------------------------------
ROUTER_CASES = [
    # (T, E, k, score, pre, groups, gtopk, scale, bias, dtype)
    (257, 8, 2, "softmax", False, None, None, None, False, torch.float32),
    (1000, 128, 8, "softmax", False, None, None, None, False, torch.float32),
    (300, 128, 8, "softmax", True, None, None, 2.0, False, torch.float32),
    (300, 128, 8, "softmax", True, None, None, None, True, torch.float32),
    (200, 256, 8, "sigmoid", False, 8, 4, 2.5, True, torch.float32),
    (200, 256, 8, "sigmoid", False, None, None, None, False, torch.float32),
    (200, 64, 6, "sqrtsoftplus", False, None, None, 1.5, False, torch.float32),
    (64, 512, 8, "softmax", True, 8, 4, 2.5, True, torch.float32),
    (77, 16, 1, "softmax", False, None, None, None, False, torch.float32),
    (77, 16, 1, "sigmoid", False, None, None, None, False, torch.float32),
    (500, 128, 8, "softmax", False, None, None, None, False, torch.bfloat16),
    # fp64 logits (moe_router_dtype "fp64"): selection on the fp64 values
    (1000, 128, 8, "softmax", False, None, None, None, False, torch.float64),
    (300, 128, 8, "softmax", True, None, None, 2.0, True, torch.float64),
    (200, 256, 8, "sigmoid", False, 8, 4, 2.5, True, torch.float64),
    (64, 512, 8, "softmax", False, 8, 4, None, False, torch.float64),
]


@pytest.mark.parametrize("case", ROUTER_CASES, ids=lambda c: f"T{c[0]}E{c[1]}k{c[2]}{c[3]}{'pre' if c[4] else ''}g{c[5]}{str(c[9])[6:]}")
def test_router_matches_oracle(hip_ops, case):
    T, E, k, score, pre, groups, gtopk, scale, use_bias, dtype = case
    g = torch.Generator().manual_seed(T * 31 + E)
    logits = torch.randn(T, E, generator=g).to(dtype)
    bias = (torch.randn(E, generator=g) * 0.05) if use_bias else None
    kwargs = dict(use_pre_softmax=pre, num_groups=groups, group_topk=gtopk, scaling_factor=scale,
                  score_function=score, expert_bias=bias)
    ref_logits = logits.clone().requires_grad_()
    probs_r, map_r, ids_r = o_route.topk_softmax_with_capacity(ref_logits, k, **kwargs)
    dev_logits = logits.to(DEV).requires_grad_()
    probs, rmap, ids = hip_ops.topk_softmax_with_capacity(
        dev_logits, k, **{**kwargs, "expert_bias": None if bias is None else bias.to(DEV)})
    exact = dtype in (torch.float32, torch.float64)
    if exact:
        # Bit-exact selection (no ties with fp32 / fp64 N(0, 1) logits).
        assert torch.equal(ids.cpu(), ids_r)
        assert torch.equal(rmap.cpu(), map_r)
    else:
        # bf16 logits tie at the k-th score for some tokens; compare the
        # selected *sets* where the k-th and (k+1)-th scores differ.
        srt = logits.float().sort(dim=1, descending=True).values
        clean = srt[:, k - 1] != srt[:, k] if k < E else torch.ones(T, dtype=torch.bool)
        assert torch.equal(rmap.cpu()[clean], map_r[clean])
        assert torch.equal(ids.cpu()[clean].sort(1).values, ids_r[clean].sort(1).values)
    assert probs.dtype == dtype
    # fp64 logits: the reference forms the probabilities in fp32 and widens them
    # (softmax(..., dtype=float32), logits.float()), so fp32 rounding is the bar.
    tol = 2e-6 if exact else 8e-3
    rows = slice(None) if exact else clean
    mx, _ = rel_errors(probs.cpu()[rows], probs_r[rows])
    assert mx <= tol, mx
    # backward through the dense probs
    w = torch.randn(T, E, generator=g).to(dtype)
    (probs_r * w).sum().backward()
    (probs * w.to(DEV)).sum().backward()
    if exact:
        assert dev_logits.grad.dtype == dtype
        mx, mean = rel_errors(dev_logits.grad.cpu(), ref_logits.grad)
        assert mx <= 1e-5 and mean <= 1e-6, (mx, mean)
    else:
        clean_rows = clean
        assert_bf16_close(dev_logits.grad.cpu()[clean_rows], ref_logits.grad[clean_rows], what="dlogits")


def test_router_fp64_selects_on_fp64_logits(hip_ops):
    """fp64 logits that differ below fp32 resolution: the reference's top-k of
    the fp64 logits (utils.py:190-196) orders them by their fp64 values, where
    fp32 keys would tie and go to the lower expert id."""
    T, E, k = 64, 32, 2
    g = torch.Generator().manual_seed(11)
    logits = torch.randn(T, E, generator=g, dtype=torch.float64) - 4.0
    base = torch.rand(T, generator=g, dtype=torch.float64) + 1.0
    lo = torch.randint(0, E // 2, (T,), generator=g)
    hi = lo + E // 2
    logits[torch.arange(T), lo] = base
    logits[torch.arange(T), hi] = base + 1e-12  # the same fp32 value, larger in fp64
    assert torch.equal(logits[torch.arange(T), lo].float(), logits[torch.arange(T), hi].float())
    probs_r, map_r, ids_r = o_route.topk_softmax_with_capacity(logits, k)
    assert torch.equal(ids_r[:, 0], hi) and torch.equal(ids_r[:, 1], lo)
    probs, rmap, ids = hip_ops.topk_softmax_with_capacity(logits.to(DEV), k)
    assert torch.equal(ids.cpu(), ids_r)
    assert torch.equal(rmap.cpu(), map_r)
    assert probs.dtype == torch.float64
    assert rel_errors(probs.cpu(), probs_r)[0] <= 2e-6


def test_router_hash_routing(hip_ops):
    T, E, k = 40, 32, 4
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(T, E, generator=g)
    table = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(10)])
    input_ids = torch.randint(0, 10, (T,), generator=g)
    for score in ("softmax", "sigmoid"):
        for pre in (False, True):
            kw = dict(use_pre_softmax=pre, score_function=score, use_hash_routing=True,
                      hash_table=table, input_ids=input_ids, scaling_factor=1.7)
            pr, mr, ir = o_route.topk_softmax_with_capacity(logits, k, **kw)
            p, m, i = hip_ops.topk_softmax_with_capacity(
                logits.to(DEV), k, **{**kw, "hash_table": table.to(DEV), "input_ids": input_ids.to(DEV)})
            assert torch.equal(i.cpu(), ir)
            assert torch.equal(m.cpu(), mr)
            assert rel_errors(p.cpu(), pr)[0] <= 2e-6


def test_router_low_precision_selection(hip_ops):
    # KAT: tests/models/test_moe_router.py:74-83
    for score in ("softmax", "sigmoid", "sqrtsoftplus"):
        for dtype in (torch.bfloat16, torch.float16):
            logits = torch.tensor([[0.0, 0.0001]], dtype=dtype, device=DEV)
            _, rmap, ids = hip_ops.topk_softmax_with_capacity(logits, 1, use_pre_softmax=True,
                                                               score_function=score)
            assert rmap.cpu().tolist() == [[False, True]]
            assert ids.cpu().tolist() == [[1]]


def test_router_ties_go_to_lower_expert(hip_ops):
    logits = torch.tensor([[1.0, 3.0, 3.0, 2.0, 3.0]], device=DEV)
    _, _, ids = hip_ops.topk_softmax_with_capacity(logits, 2)
    assert ids.cpu().tolist() == [[1, 2]]


# T, H, E, k, score, pre-softmax, groups, group_topk, scale, bias, input dtype, router dtype
GATE_CASES = [
    (1000, 2048, 128, 8, "softmax", False, None, None, None, False, torch.bfloat16, torch.float32),
    (333, 512, 256, 8, "sigmoid", False, 8, 4, 2.5, True, torch.bfloat16, torch.bfloat16),
    (100, 64, 32, 2, "sqrtsoftplus", False, None, None, None, False, torch.bfloat16, torch.float32),
    (65, 128, 160, 6, "softmax", True, None, None, 1.5, True, torch.float16, torch.float32),
    (129, 192, 64, 4, "softmax", False, None, None, None, False, torch.bfloat16, torch.bfloat16),
    (200, 256, 96, 4, "sigmoid", False, None, None, None, False, torch.float16, torch.float16),
    (0, 256, 128, 8, "softmax", False, None, None, None, False, torch.bfloat16, torch.float32),
    # 64-token blocks (the grid covers the device); the cases above use 32-token blocks
    (16448, 128, 128, 8, "softmax", False, None, None, None, False, torch.bfloat16, torch.float32),
]


@pytest.mark.parametrize("case", GATE_CASES,
                         ids=lambda c: f"T{c[0]}H{c[1]}E{c[2]}k{c[3]}{c[4]}{str(c[10])[6:]}-{str(c[11])[6:]}")
def test_router_gate_topk_matches_linear_and_router(hip_ops, case):
    """Fused gating linear + top-k (router.py:25-101, utils.py:127-230): logits
    vs the exact-product fp32 linear of the same 16-bit inputs (the order of the
    fp32 sum differs), then the oracle top-k applied to the kernel's own logits
    (bit-exact ids and map), and gradients of x and the weight vs autograd."""
    T, H, E, k, score, pre, groups, gtopk, scale, use_bias, idt, rdt = case
    g = torch.Generator().manual_seed(T * 7 + E)
    x = torch.randn(T, H, generator=g).to(idt)
    w = (torch.randn(E, H, generator=g) * H ** -0.5).to(idt)
    bias = (torch.randn(E, generator=g) * 0.05) if use_bias else None
    kw = dict(use_pre_softmax=pre, num_groups=groups, group_topk=gtopk, scaling_factor=scale,
              score_function=score, expert_bias=bias)
    xd = x.to(DEV).requires_grad_()
    wd = w.to(DEV).requires_grad_()
    probs, rmap, ids, logits = hip_ops.router_gate_topk(
        xd, wd, rdt, k, **{**kw, "expert_bias": None if bias is None else bias.to(DEV)})
    assert logits.dtype == rdt and probs.dtype == rdt and logits.shape == (T, E)
    exact = x.double() @ w.double().T
    lg = logits.detach().cpu()
    if rdt == torch.float32:
        err = (lg.double() - exact).abs().max().item() if T else 0.0
        assert err <= 1e-5 * max(1.0, exact.abs().max().item() if T else 1.0), err
    else:  # one rounding of an fp32 sum: within one bf16 step of the exact value
        assert torch.all((lg.double() - exact).abs() <= exact.abs() * 2 ** -8 + 1e-6)
    ref_lg = lg.clone().requires_grad_()
    pr, mr, ir = o_route.topk_softmax_with_capacity(ref_lg, k, **kw)
    if rdt == torch.float32:
        assert torch.equal(ids.cpu(), ir) and torch.equal(rmap.cpu(), mr)
        rows = slice(None)
    else:
        # bf16 logits tie; PyTorch's topk has no tie rule (the kernel takes the
        # lower id): compare the selected sets where the k-th and (k+1)-th
        # logits differ, as test_router_matches_oracle does
        srt = lg.float().sort(dim=1, descending=True).values
        rows = srt[:, k - 1] != srt[:, k]
        assert torch.equal(rmap.cpu()[rows], mr[rows])
        assert torch.equal(ids.cpu()[rows].sort(1).values, ir[rows].sort(1).values)
    tol = 2e-6 if rdt == torch.float32 else 8e-3
    if T:
        assert rel_errors(probs.detach().cpu()[rows], pr.detach()[rows])[0] <= tol
    # backward through probs and logits; the linear's backward as the reference forms it
    gp = torch.randn(T, E, generator=g).to(rdt)
    gl = torch.randn(T, E, generator=g).to(rdt)
    xr = x.clone().requires_grad_()
    wr = w.clone().requires_grad_()
    ((pr * gp).sum() + (ref_lg * gl).sum()).backward()
    glog = ref_lg.grad  # d loss / d logits of the reference composition
    gx_r = (glog.to(rdt) @ wr.detach().to(rdt)).to(idt)
    gw_r = (glog.to(rdt).T @ xr.detach().to(rdt)).to(idt)
    ((probs * gp.to(DEV)).sum() + (logits * gl.to(DEV)).sum()).backward()
    if T == 0:
        assert xd.grad.shape == (0, H)
        return
    if rdt != torch.float32 and not bool(rows.all()):
        return  # a tie row routes differently, so its gradient differs; selection checked above
    assert_bf16_close(xd.grad.cpu(), gx_r, what="dx")
    assert_bf16_close(wd.grad.cpu(), gw_r, what="dw")


def test_router_gate_topk_hash_routing(hip_ops):
    T, H, E, k = 40, 128, 64, 4
    g = torch.Generator().manual_seed(8)
    x = torch.randn(T, H, generator=g).bfloat16()
    w = (torch.randn(E, H, generator=g) * 0.1).bfloat16()
    table = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(10)])
    input_ids = torch.randint(0, 10, (T,), generator=g)
    kw = dict(use_pre_softmax=True, score_function="sigmoid", use_hash_routing=True,
              scaling_factor=1.7)
    p, m, i, lg = hip_ops.router_gate_topk(x.to(DEV), w.to(DEV), torch.float32, k,
                                           hash_table=table.to(DEV), input_ids=input_ids.to(DEV),
                                           **kw)
    pr, mr, ir = o_route.topk_softmax_with_capacity(lg.cpu(), k, hash_table=table,
                                                    input_ids=input_ids, **kw)
    assert torch.equal(i.cpu(), ir) and torch.equal(m.cpu(), mr)
    assert rel_errors(p.cpu(), pr)[0] <= 2e-6


def test_router_gate_rejects_unsupported_shapes(hip_ops):
    x = torch.randn(8, 96, device=DEV).bfloat16()
    w = torch.randn(64, 96, device=DEV).bfloat16()
    with pytest.raises(ValueError, match="multiple of 64"):
        hip_ops.router_gate_topk(x, w, torch.float32, 2)
    x = torch.randn(8, 128, device=DEV).bfloat16()
    w = torch.randn(48, 128, device=DEV).bfloat16()
    with pytest.raises(ValueError, match="multiple of 32"):
        hip_ops.router_gate_topk(x, w, torch.float32, 2)


# T, E, k, score function, logits dtype, padded rows
LOSS_CASES = [
    (1000, 128, 8, "softmax", torch.float32, False),
    (777, 33, 3, "sigmoid", torch.float32, True),
    (513, 256, 8, "sigmoid", torch.float32, False),
    (300, 160, 6, "sqrtsoftplus", torch.float32, True),
    (20000, 64, 4, "softmax", torch.float32, True),  # several tokens per wave
    (1024, 128, 8, "softmax", torch.bfloat16, False),
    (700, 64, 4, "sigmoid", torch.float16, True),
    (5, 1024, 1, "sigmoid", torch.float32, False),
    (0, 16, 2, "softmax", torch.float32, False),
    (1000, 128, 8, "softmax", torch.float64, False),
    (777, 33, 3, "sigmoid", torch.float64, True),
]


@pytest.mark.parametrize("case", LOSS_CASES, ids=lambda c: f"{c[0]}x{c[1]}k{c[2]}-{c[3]}-{c[4]}")
def test_router_loss_stats_matches_oracle(hip_ops, case):
    """Aux/z-loss sums (moe_utils.py:15-70) vs the oracle: counts bit-exact
    for fp32 logits, score sums and z within fp32 rounding, and the one-pass
    backward vs autograd of the oracle composition."""
    T, E, k, score, dtype, padded = case
    g = torch.Generator().manual_seed(T + 7 * E)
    logits = (torch.randn(T, E, generator=g) * 2).to(dtype)
    pad = (torch.rand(T, generator=g) < 0.2) if padded else None
    ref = logits.clone().requires_grad_()
    ps_r, cn_r, zs_r = o_route.router_loss_stats(ref, k, score, pad)
    dev = logits.to(DEV).requires_grad_()
    ps, cn, zs = hip_ops.router_loss_stats(dev, k, score, None if pad is None else pad.to(DEV))
    assert ps.dtype == torch.float32 and cn.dtype == torch.int64 and zs.dim() == 0
    n_valid = T - (int(pad.sum()) if pad is not None else 0)
    assert int(cn.sum()) == k * n_valid
    wide = dtype in (torch.float32, torch.float64)
    if wide:
        assert torch.equal(cn.cpu(), cn_r)
    else:
        # bf16 logits tie; only rows with a tie at the k-th score may differ
        s = torch.softmax(logits.float(), -1).sort(dim=1, descending=True).values
        ties = int((s[:, k - 1] == s[:, k]).sum())
        assert int((cn.cpu() - cn_r).abs().sum()) <= 2 * ties
    torch.testing.assert_close(ps.cpu(), ps_r, rtol=1e-5, atol=1e-5)
    # fp64 logits: the reference's fp64 logsumexp, here formed in fp32
    ztol = 1e-5 if wide else 2e-3
    torch.testing.assert_close(zs.cpu().to(zs_r.dtype), zs_r, rtol=ztol, atol=1e-5)
    gp = torch.randn(E, generator=g)
    gz = torch.randn((), generator=g)
    ((ps_r * gp).sum() + zs_r * gz).backward()
    ((ps * gp.to(DEV)).sum() + zs * gz.to(DEV)).backward()
    if T == 0:
        assert dev.grad.shape == (0, E)
        return
    if pad is not None:
        assert not dev.grad.cpu()[pad].any()
    if wide:
        assert dev.grad.dtype == dtype
        mx, mean = rel_errors(dev.grad.cpu(), ref.grad)
        assert mx <= 2e-5 and mean <= 2e-6, (mx, mean)
    else:
        assert_bf16_close(dev.grad.cpu(), ref.grad, what="dlogits")


def test_router_loss_stats_match_golden_brute_force(hip_ops):
    """tests/golden/router_loss_cases.json (per-row brute force in Python floats,
    padding rows included) through the HIP kernels."""
    import json
    import os

    path = os.path.join(os.path.dirname(__file__), "golden", "router_loss_cases.json")
    with open(path) as f:
        cases = json.load(f)
    for c in cases:
        logits = torch.tensor(c["logits"], dtype=torch.float32, device=DEV)
        pad = torch.tensor(c["padding_mask"], dtype=torch.bool, device=DEV)
        ps, cn, zs = hip_ops.router_loss_stats(logits, c["k"], c["score_function"], pad)
        torch.testing.assert_close(ps.cpu().double(), torch.tensor(c["prob_sum"], dtype=torch.float64),
                                   rtol=1e-5, atol=1e-6)
        assert cn.cpu().tolist() == c["tokens_per_expert"]
        torch.testing.assert_close(zs.cpu().double(), torch.tensor(c["z_sum"], dtype=torch.float64),
                                   rtol=1e-5, atol=1e-6)


def test_router_loss_stats_is_reproducible(hip_ops):
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(50000, 128, generator=g).to(DEV)
    a = hip_ops.router_loss_stats(logits, 8, "softmax")
    b = hip_ops.router_loss_stats(logits, 8, "softmax")
    for x, y in zip(a, b):
        assert torch.equal(x, y)


@pytest.mark.parametrize("router_dtype", ["fp32", "fp64"])
def test_router_aux_and_z_losses_on_gpu_match_cpu(process_ops, monkeypatch, router_dtype):
    """TopKRouter with both losses (router.py:164-356) through the HIP ops vs the
    same router on the CPU oracle: probs, loss metrics, weight and input grads;
    fp32 and fp64 router dtypes (router.py:97-100)."""
    from torchturbo_amd.moe import MoEConfig, TopKRouter
    from torchturbo_amd.moe.router import MoEAuxLossAutoScaler
    from torchturbo_amd.runtime import CpuRuntime, CudaRuntime

    monkeypatch.setattr(MoEAuxLossAutoScaler, "loss_scale", 1.0)
    # seed 4: every token's 8th and 9th logits differ by >= 2.8e-4, far above
    # the rounding difference of the CPU and GPU fp32 gating GEMMs
    torch.manual_seed(4)
    cfg = MoEConfig(hidden_size=64, num_moe_experts=128, moe_router_topk=8,
                    moe_router_dtype=router_dtype, moe_aux_loss_coeff=0.01,
                    moe_z_loss_coeff=0.001, params_dtype=torch.float32)
    router = TopKRouter(cfg)
    torch.nn.init.normal_(router.weight, std=0.2)
    x = torch.randn(4, 128, 64)
    w = torch.randn(512, 128)

    process_ops(CpuRuntime(), OpPolicy.NATIVE, oracle=True)
    xr = x.clone().requires_grad_()
    pr, mr, _, _ = router(xr)
    (pr * w).sum().backward()
    m_ref = router.pop_metrics()
    gw_ref = router.weight.grad.clone()

    process_ops(CudaRuntime(), OpPolicy.CUSTOM)
    router = router.to(DEV)
    router.weight.grad = None
    xd = x.to(DEV).requires_grad_()
    pd, md, _, _ = router(xd)
    (pd * w.to(DEV)).sum().backward()
    m = router.pop_metrics()
    assert torch.equal(md.cpu(), mr)
    torch.testing.assert_close(pd.cpu(), pr, rtol=1e-5, atol=1e-6)
    for key in ("aux_loss", "aux_loss_scaled", "z_loss", "z_loss_scaled"):
        torch.testing.assert_close(m[key].cpu(), m_ref[key], rtol=1e-5, atol=0)
    mx, _ = rel_errors(router.weight.grad.cpu(), gw_ref)
    assert mx <= 1e-4, mx
    mx, _ = rel_errors(xd.grad.cpu(), xr.grad)
    assert mx <= 1e-4, mx


# ---------------------------------------------------------------------------
# Routing index + permutation
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("T,E,k,skew", [(1, 4, 1, False), (255, 8, 2, False), (256, 8, 2, True),
                                        (1000, 128, 8, True), (3000, 256, 8, False),
                                        (513, 64, 16, True), (100, 1000, 3, False),
                                        (77, 33, 3, True), (300, 1500, 4, False)])
def test_route_index_bit_exact(T, E, k, skew):
    """Counting-sort row map vs the brute-force oracle; E = 33 (odd: the lane-mask
    table's alignment) and E = 1500 (above the lane-mask limit: one ballot per expert)."""
    from torchturbo_amd.providers.hip._functions import route_index

    ids = distinct_ids(T, E, k, seed=T + E, skew=skew)
    probs = torch.rand(T, E)
    rows, tor, pprobs, counts = route_index(ids.to(DEV), E, probs.to(DEV))
    r_rows, r_tor, r_counts, _ = route_np.route_index(ids.numpy(), E)
    assert np.array_equal(rows.cpu().numpy(), r_rows)
    assert np.array_equal(tor.cpu().numpy(), r_tor)
    assert np.array_equal(counts.cpu().numpy(), r_counts)
    order = np.argsort(ids.reshape(-1).numpy(), kind="stable")
    flat_ids = ids.reshape(-1).numpy()[order]
    expected_probs = probs.numpy()[order // k, flat_ids]
    assert np.array_equal(pprobs.cpu().numpy(), expected_probs)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
# wide rows: one thread per 16-byte vector up to 1024 (H 4096: 512 threads; H 5000:
# 625 vectors, idle threads; H 9216: more vectors than threads)
@pytest.mark.parametrize("T,H,E,k", [(300, 256, 8, 2), (517, 136, 64, 6), (64, 2048, 128, 8),
                                     (40, 4096, 8, 2), (33, 5000, 8, 3), (24, 9216, 16, 8)])
def test_permutation_and_unpermutation_bit_exact(hip_ops, dtype, T, H, E, k):
    g = torch.Generator().manual_seed(T + H)
    ids = distinct_ids(T, E, k, seed=T)
    rmap = torch.zeros(T, E, dtype=torch.bool).scatter(1, ids, True)
    x = torch.randn(T, H, generator=g).to(dtype)
    probs = torch.rand(T, E, generator=g) * rmap
    ref = o_perm.permute(x, rmap, probs=probs, expert_indices=ids)
    got = hip_ops.moe_permutation(x.to(DEV), rmap.to(DEV), probs=probs.to(DEV),
                                  expert_indices=ids.to(DEV))
    assert torch.equal(got.row_indices.cpu(), ref.row_indices)
    assert torch.equal(got.tokens.cpu(), ref.tokens)
    assert torch.equal(got.probs.cpu(), ref.probs)
    assert torch.equal(got.tokens_per_expert.cpu(), rmap.sum(0))
    # unpermutation of arbitrary expert outputs: unweighted and weighted
    y = torch.randn(T * k, H, generator=g).to(dtype)
    for w in (None, probs, probs.to(torch.bfloat16)):
        perm_r = MoEPermutation(y, None, ref.row_indices, ids)
        perm_g = MoEPermutation(y.to(DEV), None, got.row_indices, ids.to(DEV))
        out_r = o_perm.unpermute(perm_r, torch.Size([T, H]), probs=w)
        out_g = hip_ops.moe_unpermutation(perm_g, torch.Size([T, H]),
                                          probs=None if w is None else w.to(DEV))
        assert out_g.dtype == out_r.dtype
        assert torch.equal(out_g.cpu(), out_r), f"weights={None if w is None else w.dtype}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_permutation_backward(hip_ops, dtype):
    T, H, E, k = 200, 128, 16, 4
    g = torch.Generator().manual_seed(3)
    ids = distinct_ids(T, E, k, seed=9)
    rmap = torch.zeros(T, E, dtype=torch.bool).scatter(1, ids, True)
    x = torch.randn(T, H, generator=g).to(dtype)
    probs = torch.rand(T, E, generator=g) * rmap
    gy = torch.randn(T * k, H, generator=g).to(dtype)
    gp = torch.randn(T * k, generator=g)
    xr, pr = x.clone().requires_grad_(), probs.clone().requires_grad_()
    ref = o_perm.permute(xr, rmap, probs=pr, expert_indices=ids)
    torch.autograd.backward([ref.tokens, ref.probs], [gy, gp])
    xd, pd = x.to(DEV).requires_grad_(), probs.to(DEV).requires_grad_()
    got = hip_ops.moe_permutation(xd, rmap.to(DEV), probs=pd, expert_indices=ids.to(DEV))
    torch.autograd.backward([got.tokens, got.probs], [gy.to(DEV), gp.to(DEV)])
    assert torch.equal(xd.grad.cpu(), xr.grad)  # fp32 gather-sum in row order
    assert torch.equal(pd.grad.cpu(), pr.grad)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_unpermutation_backward(hip_ops, dtype):
    T, H, E, k = 150, 192, 12, 3
    g = torch.Generator().manual_seed(4)
    ids = distinct_ids(T, E, k, seed=2)
    rmap = torch.zeros(T, E, dtype=torch.bool).scatter(1, ids, True)
    rows = o_perm.permute(torch.zeros(T, 1), rmap, expert_indices=ids).row_indices
    y = torch.randn(T * k, H, generator=g).to(dtype)
    probs = torch.rand(T, E, generator=g)
    go = torch.randn(T, H, generator=g).to(dtype)
    for weighted in (False, True):
        yr = y.clone().requires_grad_()
        pr = probs.clone().requires_grad_() if weighted else None
        out_r = o_perm.unpermute(MoEPermutation(yr, None, rows, ids), torch.Size([T, H]), probs=pr)
        out_r.backward(go)
        yd = y.to(DEV).requires_grad_()
        pd = probs.to(DEV).requires_grad_() if weighted else None
        out_d = hip_ops.moe_unpermutation(MoEPermutation(yd, None, rows.to(DEV), ids.to(DEV)),
                                          torch.Size([T, H]), probs=pd)
        out_d.backward(go.to(DEV))
        assert torch.equal(yd.grad.cpu(), yr.grad)
        if weighted:
            mx, mean = rel_errors(pd.grad.cpu(), pr.grad)
            assert mx <= 1e-5 and mean <= 1e-6, (mx, mean)


def test_permutation_kats(hip_ops):
    # tests/ops/test_moe_permutation_contract.py:72-84
    r = hip_ops.moe_permutation(torch.tensor([[2.0], [3.0]], device=DEV),
                                torch.tensor([[False, True], [True, False]], device=DEV),
                                probs=torch.tensor([[0.0, 0.5], [0.25, 0.0]], device=DEV))
    assert r.tokens.cpu().tolist() == [[3.0], [2.0]]
    assert r.probs.cpu().tolist() == [0.25, 0.5]
    assert r.row_indices.cpu().tolist() == [[1], [0]]
    # :307-370 (mixed providers case, custom both sides)
    tokens = torch.tensor([[10.0], [20.0], [30.0]], device=DEV, requires_grad=True)
    probs = torch.tensor([[0.25, 0.0, 0.5], [0.0, 0.75, 0.125], [0.125, 0.25, 0.0]],
                         device=DEV, requires_grad=True)
    mask = probs.detach().bool()
    idx = torch.tensor([[0, 2], [1, 2], [0, 1]], device=DEV)
    m = hip_ops.moe_permutation(tokens, mask, probs=probs, expert_indices=idx)
    assert m.tokens.detach().cpu().flatten().tolist() == [10.0, 30.0, 20.0, 30.0, 10.0, 20.0]
    assert m.row_indices.cpu().tolist() == [[0, 4], [2, 5], [1, 3]]
    out = hip_ops.moe_unpermutation(m, tokens.shape, probs=probs)
    assert out.detach().cpu().flatten().tolist() == [7.5, 17.5, 11.25]
    out.sum().backward()
    assert tokens.grad.cpu().flatten().tolist() == probs.detach().sum(1).cpu().tolist()
    torch.testing.assert_close(probs.grad.cpu(), (tokens.detach().expand_as(probs) * mask).cpu())
    un = hip_ops.moe_unpermutation(m, tokens.shape)
    assert un.detach().cpu().flatten().tolist() == [20.0, 40.0, 60.0]
    # :412-434 probability precision is retained
    packed = torch.tensor([[1.0], [-1.0]], dtype=torch.bfloat16, device=DEV, requires_grad=True)
    p = torch.tensor([[1.00390625, 1.0]], device=DEV, requires_grad=True)
    mp = MoEPermutation(packed, None, torch.tensor([[0, 1]], dtype=torch.int32, device=DEV),
                        torch.tensor([[0, 1]], device=DEV))
    o = hip_ops.moe_unpermutation(mp, torch.Size([1, 1]), probs=p)
    assert o.dtype == torch.bfloat16 and o.item() == 0.00390625
    o.sum().backward()
    assert p.grad.cpu().tolist() == [[1.0, -1.0]]
    # :37-69 small contributions survive (fp32 accumulation), bf16 and fp16
    for dtype, large in ((torch.bfloat16, 256), (torch.float16, 2048)):
        packed = torch.tensor([[large], [-large], [1], [2], [-large], [large]], dtype=dtype, device=DEV)
        mp = MoEPermutation(packed, None, torch.tensor([[0, 2, 4], [5, 1, 3]], dtype=torch.int32, device=DEV),
                            torch.tensor([[0, 1, 2], [2, 0, 1]], device=DEV))
        o = hip_ops.moe_unpermutation(mp, torch.Size([2, 1]))
        assert o.cpu().float().flatten().tolist() == [1.0, 2.0]


def test_sort_chunks_kats(hip_ops):
    """tests/models/test_moe_permutation.py:125-130 and :133-151 (an empty chunk, probs,
    gradients, and the inverse order restoring the input), on the GPU."""
    tokens = torch.tensor([[10.0], [20.0], [30.0]], device=DEV)
    out, _ = hip_ops.moe_sort_chunks(tokens, torch.tensor([1, 2], device=DEV),
                                     torch.tensor([1, 0], device=DEV))
    assert out.cpu().tolist() == [[20.0], [30.0], [10.0]]
    for n in (0, 3):
        tokens = torch.tensor([[10.0], [20.0], [30.0]], device=DEV)[:n].requires_grad_()
        probs = torch.tensor([0.1, 0.2, 0.3], device=DEV)[:n].requires_grad_()
        sizes = torch.tensor([2, 0, 1] if n else [0, 0, 0], device=DEV)
        order = torch.tensor([2, 0, 1], device=DEV)
        output, weights = hip_ops.moe_sort_chunks(tokens, sizes, order, probs=probs)
        rows = torch.tensor([2, 0, 1] if n else [], dtype=torch.long, device=DEV)
        assert torch.equal(output, tokens[rows])
        restored, _ = hip_ops.moe_sort_chunks(output, sizes[order], order.argsort())
        assert torch.equal(restored, tokens)
        (output * weights[:, None]).sum().backward()
        assert torch.equal(tokens.grad.flatten(), probs.detach())
        assert torch.equal(probs.grad, tokens.detach().flatten())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("C,H,max_rows", [(8, 256, 300), (128, 2048, 96), (33, 5000, 40),
                                          (4096, 64, 12), (64, 1, 50)])
def test_sort_chunks_matches_oracle(hip_ops, dtype, C, H, max_rows):
    """Random chunk sizes (empty chunks included) and orders, among them the EP
    exchange's (rank, expert) -> (expert, rank) transpose; rows, probs and both
    gradients bit-exact against the oracle (a pure data movement)."""
    g = torch.Generator().manual_seed(C + H)
    sizes = torch.randint(0, max_rows + 1, (C,), generator=g)
    sizes[C // 2] = 0
    if C == 128:  # 8 ranks x 16 local experts, regrouped by expert
        order = torch.arange(C).view(8, 16).t().reshape(-1)
    else:
        order = torch.randperm(C, generator=g)
    rows = int(sizes.sum())
    x = torch.randn(rows, H, generator=g).to(dtype)
    if H == 1:
        x = x.view(rows)
    p = torch.rand(rows, generator=g)
    gx = torch.randn(x.shape, generator=g).to(dtype)
    gp = torch.randn(rows, generator=g)
    xr, pr = x.clone().requires_grad_(), p.clone().requires_grad_()
    out_r, outp_r = o_perm.sort_chunks(xr, sizes, order, probs=pr)
    torch.autograd.backward([out_r, outp_r], [gx, gp])
    xd, pd = x.to(DEV).requires_grad_(), p.to(DEV).requires_grad_()
    out_d, outp_d = hip_ops.moe_sort_chunks(xd, sizes.to(DEV), order.to(DEV), probs=pd)
    torch.autograd.backward([out_d, outp_d], [gx.to(DEV), gp.to(DEV)])
    assert torch.equal(out_d.cpu(), out_r.detach())
    assert torch.equal(outp_d.cpu(), outp_r.detach())
    assert torch.equal(xd.grad.cpu(), xr.grad)
    assert torch.equal(pd.grad.cpu(), pr.grad)
    # the inverse order restores the input
    back, _ = hip_ops.moe_sort_chunks(out_d.detach(), sizes[order].to(DEV), order.argsort().to(DEV))
    assert torch.equal(back.cpu(), x)


def test_sort_chunks_rejects_inconsistent_metadata(hip_ops):
    from torchturbo_amd import checks

    x = torch.randn(10, 4, device=DEV)
    with pytest.raises(ValueError, match="chunk ids"):
        hip_ops.moe_sort_chunks(x, torch.tensor([5, 5], device=DEV), torch.tensor([0], device=DEV))
    with pytest.raises(ValueError, match="input device"):
        hip_ops.moe_sort_chunks(x, torch.tensor([5, 5]), torch.tensor([1, 0], device=DEV))
    with checks.checking():
        with pytest.raises(ValueError, match="sum to 9"):
            hip_ops.moe_sort_chunks(x, torch.tensor([5, 4], device=DEV),
                                    torch.tensor([1, 0], device=DEV))
        with pytest.raises(ValueError, match="permutation"):
            hip_ops.moe_sort_chunks(x, torch.tensor([5, 5], device=DEV),
                                    torch.tensor([1, 1], device=DEV))
        out, _ = hip_ops.moe_sort_chunks(x, torch.tensor([6, 4], device=DEV),
                                         torch.tensor([1, 0], device=DEV))
        assert torch.equal(out, torch.cat([x[6:], x[:6]]))


def test_routing_ids_out_of_range_or_repeated(hip_ops):
    """Bad routing input. With checks on: ValueError, as the reference's gather and
    top-k checks raise (ops/moe.py:62-65, native/moe_permutation.py:52-56). With checks
    off: the rejected slots get row -1, no packed row and no count; every accepted slot
    keeps the reference's expert-major, token-ascending row."""
    from torchturbo_amd import checks

    T, H, E, k = 64, 32, 8, 3
    ids = distinct_ids(T, E, k, seed=5)
    rmap = torch.zeros(T, E, dtype=torch.bool).scatter(1, ids, True)
    x = torch.randn(T, H)
    bad = ids.clone()
    bad[5, 1] = E          # out of range
    bad[9, 0] = -1         # out of range
    bad[12, 2] = bad[12, 0]  # repeated within the token
    with checks.checking():
        with pytest.raises(ValueError, match="3 of 192 slots"):
            hip_ops.moe_permutation(x.to(DEV), rmap.to(DEV), expert_indices=bad.to(DEV))
        other = ids.clone()
        free = [e for e in range(E) if e not in ids[3].tolist()][0]
        other[3, 0] = free   # valid, distinct, but not what routing_map selects
        with pytest.raises(ValueError, match="disagree for 1 of 64 tokens"):
            hip_ops.moe_permutation(x.to(DEV), rmap.to(DEV), expert_indices=other.to(DEV))
        ok = hip_ops.moe_permutation(x.to(DEV), rmap.to(DEV), expert_indices=ids.to(DEV))
        assert int(ok.tokens_per_expert.sum()) == T * k
    got = hip_ops.moe_permutation(x.to(DEV), rmap.to(DEV), expert_indices=bad.to(DEV))
    rows = got.row_indices.cpu()
    rejected = {(5, 1), (9, 0), (12, 2)}
    accepted = sorted((int(bad[t, j]), t, j) for t in range(T) for j in range(k)
                      if (t, j) not in rejected)
    expect = torch.full((T, k), -1, dtype=torch.int32)
    for r, (_, t, j) in enumerate(accepted):
        expect[t, j] = r
    assert torch.equal(rows, expect)
    assert int(got.tokens_per_expert.sum()) == T * k - 3
    assert torch.equal(got.tokens[:len(accepted)].cpu(), x[[t for _, t, _ in accepted]])
    # the combine skips rejected slots: token t gets (accepted slots of t) * x[t]
    out = hip_ops.moe_unpermutation(got, torch.Size([T, H])).cpu()
    n_ok = torch.tensor([sum((t, j) not in rejected for j in range(k)) for t in range(T)])
    assert torch.equal(out, x * n_ok[:, None].float())


def test_permutation_empty_and_zero_weight(hip_ops):
    tokens = torch.empty(0, 4, device=DEV, requires_grad=True)
    probs = torch.empty(0, 3, device=DEV, requires_grad=True)
    m = hip_ops.moe_permutation(tokens, probs.detach().bool(), probs=probs,
                                expert_indices=torch.empty(0, 2, dtype=torch.long, device=DEV))
    out = hip_ops.moe_unpermutation(m, tokens.shape, probs)
    out.sum().backward()
    assert out.shape == (0, 4)
    # zero-probability selections keep their rows and router gradient
    t = torch.tensor([[2.0]], device=DEV)
    p = torch.tensor([[0.0, 1.0]], device=DEV, requires_grad=True)
    r = hip_ops.moe_permutation(t, torch.tensor([[True, True]], device=DEV), probs=p,
                                expert_indices=torch.tensor([[0, 1]], device=DEV))
    assert r.tokens.cpu().tolist() == [[2.0], [2.0]]
    (r.tokens * r.probs[:, None]).sum().backward()
    assert p.grad.cpu().tolist() == [[2.0, 2.0]]


def test_permute_unpermute_round_trip_full_qwen_size(hip_ops):
    """Size-independent property at the Qwen3 shape: unpermute(permute(x)) == k * x."""
    from torchturbo_amd.configs import QWEN3, make_logits

    T, H, E, k = QWEN3.tokens, QWEN3.hidden, QWEN3.experts, QWEN3.topk
    logits = make_logits(QWEN3)
    _, rmap_r, ids_r = o_route.topk_softmax_with_capacity(logits, k)
    probs, rmap, ids = hip_ops.topk_softmax_with_capacity(logits.to(DEV), k)
    assert torch.equal(ids.cpu(), ids_r)
    x = torch.randn(T, H, device=DEV).to(torch.bfloat16)
    m = hip_ops.moe_permutation(x, rmap, probs=probs, expert_indices=ids)
    r_rows, _, r_counts, _ = route_np.route_index(ids_r.numpy(), E)
    assert np.array_equal(m.row_indices.cpu().numpy(), r_rows)
    assert np.array_equal(m.tokens_per_expert.cpu().numpy(), r_counts)
    back = hip_ops.moe_unpermutation(m, x.shape)
    assert torch.equal(back, (x.float() * k).to(torch.bfloat16))


# ---------------------------------------------------------------------------
# SwiGLU (+ probs)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("with_probs", [False, True])
@pytest.mark.parametrize("rows,F", [(333, 96), (129, 1000)])  # 1000: an odd count of 16-byte vectors
def test_swiglu_matches_oracle(hip_ops, dtype, with_probs, rows, F):
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(rows, 2 * F, generator=g) * 2).to(dtype)
    p = torch.rand(rows, generator=g)
    go = torch.randn(rows, F, generator=g).to(dtype)
    xr = x.clone().requires_grad_()
    pr = p.clone().requires_grad_()
    ref = o_swiglu.swiglu_probs(xr, pr) if with_probs else o_swiglu.swiglu(xr)
    ref.backward(go)
    xd = x.to(DEV).requires_grad_()
    pd = p.to(DEV).requires_grad_()
    got = hip_ops.swiglu_probs(xd, pd) if with_probs else hip_ops.swiglu(xd)
    got.backward(go.to(DEV))
    assert got.dtype == ref.dtype
    if dtype == torch.float32:
        assert rel_errors(got.cpu(), ref)[0] <= 1e-6
        assert rel_errors(xd.grad.cpu(), xr.grad)[0] <= 1e-5
    else:
        # at most one ulp away where exp() differs in the last fp32 bit
        assert_bf16_close(got.cpu(), ref, max_rel=8e-3, mean_rel=1e-4, what="swiglu")
        assert_bf16_close(xd.grad.cpu(), xr.grad, max_rel=1e-2, mean_rel=1e-3, what="dx")
    if with_probs:
        mx, mean = rel_errors(pd.grad.cpu(), pr.grad)
        assert mx <= 1e-3 and mean <= 1e-4, (mx, mean)


@pytest.mark.parametrize("act", ["silu", "gelu"])
@pytest.mark.parametrize("limit,after", [(0.0, False), (2.5, False), (2.5, True)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("with_probs", [False, True])
def test_gated_activation_matches_oracle(hip_ops, act, limit, after, dtype, with_probs):
    """GELU / capped gates (gated_activation.py:15-44) with the probability product:
    values span the cap (|x| up to ~9) so both clamped and free branches occur."""
    fn = F.silu if act == "silu" else F.gelu
    rows, Fd = 257, 80
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(rows, 2 * Fd, generator=g) * 3).to(dtype)
    p = torch.rand(rows, generator=g)
    go = torch.randn(rows, Fd, generator=g).to(dtype)
    kw = dict(activation_func=fn, limit=limit, clamp_gate_after_activation=after)
    xr = x.clone().requires_grad_()
    pr = p.clone().requires_grad_()
    ref = (o_gated.gated_activation_probs(xr, pr, **kw) if with_probs
           else o_gated.gated_activation(xr, **kw))
    ref.backward(go)
    xd = x.to(DEV).requires_grad_()
    pd = p.to(DEV).requires_grad_()
    got = (hip_ops.gated_activation_probs(xd, pd, **kw) if with_probs
           else hip_ops.gated_activation(xd, **kw))
    got.backward(go.to(DEV))
    assert got.dtype == ref.dtype and got.shape == ref.shape
    if dtype == torch.float32:
        assert rel_errors(got.cpu(), ref)[0] <= 1e-5
        assert rel_errors(xd.grad.cpu(), xr.grad)[0] <= 1e-5
    else:
        assert_bf16_close(got.cpu(), ref, max_rel=8e-3, mean_rel=1e-4, what="gated")
        assert_bf16_close(xd.grad.cpu(), xr.grad, max_rel=1e-2, mean_rel=1e-3, what="dx")
    if with_probs:
        mx, mean = rel_errors(pd.grad.cpu(), pr.grad)
        assert mx <= 1e-3 and mean <= 1e-4, (mx, mean)


def test_gated_activation_rejects_like_reference(hip_ops):
    x = torch.randn(4, 8, device=DEV)
    with pytest.raises(ValueError, match="only supports F.silu and F.gelu"):
        hip_ops.gated_activation(x, activation_func=torch.tanh)
    with pytest.raises(ValueError, match="limit must be non-negative"):
        hip_ops.gated_activation(x, activation_func=F.silu, limit=-1.0)


# ---------------------------------------------------------------------------
# Grouped GEMM
# ---------------------------------------------------------------------------
def _ref_gmm(x, w, counts, trans_b):
    return o_gmm.grouped_matmul(x.double(), w.double(), counts, trans_b=trans_b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize("counts,K,N", [([0, 5, 0, 11], 64, 32), ([300, 0, 17, 513, 1], 256, 384),
                                        ([1024] * 4, 512, 768), ([0, 0, 0], 128, 128)])
def test_grouped_matmul_fwd_bwd(hip_ops, dtype, trans_b, counts, K, N):
    g = torch.Generator().manual_seed(sum(counts) + K)
    E = len(counts)
    M = sum(counts)
    x = torch.randn(M, K, generator=g).to(dtype)
    w = (torch.randn(E, N, K, generator=g) if trans_b else torch.randn(E, K, N, generator=g)).mul(0.05).to(dtype)
    dy = torch.randn(M, N, generator=g).to(dtype)
    xr = x.double().requires_grad_()
    wr = w.double().requires_grad_()
    yr = o_gmm.grouped_matmul(xr, wr, counts, trans_b=trans_b)
    if M:  # the native op returns a graph-less [0, N] tensor when every expert is empty
        yr.backward(dy.double())
    xd = x.to(DEV).requires_grad_()
    wd = w.to(DEV).requires_grad_()
    for cnt in (counts, torch.tensor(counts), torch.tensor(counts, device=DEV)):
        xd.grad = None
        wd.grad = None
        y = hip_ops.grouped_matmul(xd, wd, cnt, trans_b=trans_b)
        y.backward(dy.to(DEV))
        assert y.shape == (M, N) and y.dtype == dtype
        if M == 0:
            assert torch.count_nonzero(wd.grad) == 0
            continue
        tol = (1e-5, 1e-6) if dtype == torch.float32 else (1e-2, 2e-3)
        for a, b, name in ((y, yr, "y"), (xd.grad, xr.grad, "dx"), (wd.grad, wr.grad, "dw")):
            mx, mean = rel_errors(a.cpu(), b)
            assert mx <= tol[0] and mean <= tol[1], f"{name}: {mx:.3e} {mean:.3e}"
        for e, c in enumerate(counts):
            if c == 0:
                assert torch.count_nonzero(wd.grad[e]) == 0


def test_grouped_matmul_integer_exact(hip_ops):
    """Small-integer operands: every product and partial sum is exact in fp32,
    so the bf16 output is the exact product rounded once (fwd, dgrad, wgrad)."""
    g = torch.Generator().manual_seed(11)
    counts = [37, 0, 300, 99]
    M, K, N = sum(counts), 256, 264
    x = torch.randint(-3, 4, (M, K), generator=g).to(torch.bfloat16)
    w = torch.randint(-3, 4, (4, K, N), generator=g).to(torch.bfloat16)
    dy = torch.randint(-3, 4, (M, N), generator=g).to(torch.bfloat16)
    xd, wd = x.to(DEV).requires_grad_(), w.to(DEV).requires_grad_()
    y = hip_ops.grouped_matmul(xd, wd, counts)
    y.backward(dy.to(DEV))
    xr, wr = x.double().requires_grad_(), w.double().requires_grad_()
    yr = o_gmm.grouped_matmul(xr, wr, counts)
    yr.backward(dy.double())
    assert torch.equal(y.cpu(), yr.to(torch.bfloat16))
    assert torch.equal(xd.grad.cpu(), xr.grad.to(torch.bfloat16))
    assert torch.equal(wd.grad.cpu(), wr.grad.to(torch.bfloat16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("E,rows", [(5, 150), (5, 1100), (13, 900), (16, 40)])
@pytest.mark.parametrize("trans_b", [False, True])
def test_grouped_matmul_wgrad_writes_every_tile(dtype, E, rows, trans_b):
    """tt_gmm_wgrad into a NaN-filled output: every expert's whole gradient is written
    (empty experts get zeros), whatever the kernel (fp32, persistent short-reduction,
    one tile per block on XCD pairs) and whether E is a multiple of 8."""
    from torchturbo_amd import _lib

    torch.backends.cuda.matmul.allow_tf32 = False
    g = torch.Generator().manual_seed(E * 1000 + rows)
    counts = torch.randint(0, 2 * rows, (E,), generator=g)
    counts[1] = 0
    M, K, N = int(counts.sum()), 512, 768
    x = torch.randint(-2, 3, (M, K), generator=g).to(dtype).to(DEV)
    dy = torch.randint(-2, 3, (M, N), generator=g).to(dtype).to(DEV)
    dw = torch.full((E, N, K) if trans_b else (E, K, N), float("nan"), dtype=dtype, device=DEV)
    cnt = counts.to(DEV)
    _lib.call("tt_gmm_wgrad", _lib.ptr(x), _lib.ptr(dy), _lib.dtype_code(dtype), M, K, N, E,
              int(trans_b), _lib.ptr(cnt), _lib.ptr(dw), _lib.stream())
    torch.cuda.synchronize()
    xs = torch.split(x.float(), counts.tolist())
    ds = torch.split(dy.float(), counts.tolist())
    for e in range(E):
        ref = xs[e].t() @ ds[e]  # [K, N]; integer sums, exact in fp32
        ref = (ref.t() if trans_b else ref).to(dtype)
        assert torch.equal(dw[e], ref), (e, int(counts[e]))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("E", [5, 13])
@pytest.mark.parametrize("K,N", [(512, 768), (64, 64)])
@pytest.mark.parametrize("trans_b", [False, True])
def test_grouped_matmul_fwd_dgrad_write_every_row(dtype, E, K, N, trans_b):
    """tt_gmm_fwd / tt_gmm_dgrad into NaN-filled outputs with small-integer operands:
    every row of every expert is written, exactly (64-deep persistent kernel for
    reductions above 64, the one-tile kernel for 64, fp32; partial and empty experts)."""
    from torchturbo_amd import _lib

    g = torch.Generator().manual_seed(E * 7 + K)
    counts = torch.randint(0, 700, (E,), generator=g)
    counts[2] = 0
    counts[3] = 1
    M = int(counts.sum())
    x = torch.randint(-2, 3, (M, K), generator=g).to(dtype).to(DEV)
    dy = torch.randint(-2, 3, (M, N), generator=g).to(dtype).to(DEV)
    wshape = (E, N, K) if trans_b else (E, K, N)
    w = torch.randint(-2, 3, wshape, generator=g).to(dtype).to(DEV)
    y = torch.full((M, N), float("nan"), dtype=dtype, device=DEV)
    dx = torch.full((M, K), float("nan"), dtype=dtype, device=DEV)
    cnt = counts.to(DEV)
    args = (_lib.dtype_code(dtype), M, K, N, E, int(trans_b), _lib.ptr(cnt))
    _lib.call("tt_gmm_fwd", _lib.ptr(x), _lib.ptr(w), *args, _lib.ptr(y), _lib.stream())
    _lib.call("tt_gmm_dgrad", _lib.ptr(dy), _lib.ptr(w), *args, _lib.ptr(dx), _lib.stream())
    torch.cuda.synchronize()
    wf = w.float()
    yr, dxr, s0 = torch.empty(M, N, device=DEV), torch.empty(M, K, device=DEV), 0
    for e, c in enumerate(counts.tolist()):
        we = wf[e].t() if trans_b else wf[e]  # [K, N]
        yr[s0:s0 + c] = x[s0:s0 + c].float() @ we
        dxr[s0:s0 + c] = dy[s0:s0 + c].float() @ we.t()
        s0 += c
    assert torch.equal(y, yr.to(dtype))
    assert torch.equal(dx, dxr.to(dtype))


@pytest.mark.parametrize("E", [5, 13])
@pytest.mark.parametrize("K,N", [(512, 768), (64, 64)])
def test_grouped_matmul_fp8_write_every_row(E, K, N):
    """tt_gmm_fp8_fwd / _dgrad into NaN-filled outputs: e4m3 weights holding small
    integers with unit block scales, so every output is an exact integer sum (the
    persistent 128x512 kernel for reductions above 64, the 256x256 kernel for 64)."""
    from torchturbo_amd import _lib

    g = torch.Generator().manual_seed(E * 11 + K)
    counts = torch.randint(0, 700, (E,), generator=g)
    counts[2] = 0
    counts[3] = 1
    M = int(counts.sum())
    x = torch.randint(-2, 3, (M, K), generator=g).to(torch.bfloat16).to(DEV)
    dy = torch.randint(-2, 3, (M, N), generator=g).to(torch.bfloat16).to(DEV)
    wq = torch.randint(-2, 3, (E, N, K), generator=g).float()
    q = wq.to(torch.float8_e4m3fn).to(DEV)
    sc = torch.ones(E, (N + 127) // 128, (K + 127) // 128, dtype=torch.bfloat16, device=DEV)
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    dx = torch.full((M, K), float("nan"), dtype=torch.bfloat16, device=DEV)
    cnt = counts.to(DEV)
    bf = _lib.dtype_code(torch.bfloat16)
    _lib.call("tt_gmm_fp8_fwd", _lib.ptr(x), _lib.ptr(q), _lib.ptr(sc), bf, M, K, N, E,
              _lib.ptr(cnt), _lib.ptr(y), _lib.stream())
    _lib.call("tt_gmm_fp8_dgrad", _lib.ptr(dy), _lib.ptr(q), _lib.ptr(sc), bf, M, K, N, E,
              _lib.ptr(cnt), _lib.ptr(dx), _lib.stream())
    torch.cuda.synchronize()
    wd = wq.to(DEV)
    yr, dxr, s0 = torch.empty(M, N, device=DEV), torch.empty(M, K, device=DEV), 0
    for e, c in enumerate(counts.tolist()):
        yr[s0:s0 + c] = x[s0:s0 + c].float() @ wd[e].t()
        dxr[s0:s0 + c] = dy[s0:s0 + c].float() @ wd[e]
        s0 += c
    assert torch.equal(y, yr.to(torch.bfloat16))
    assert torch.equal(dx, dxr.to(torch.bfloat16))


def _zipf_counts(E, M, seed, empty=(3, 17)):
    """Zipf(1.1)-skewed expert loads summing to M, with some empty experts."""
    g = torch.Generator().manual_seed(seed)
    rank = torch.randperm(E, generator=g).double() + 1.0
    p = rank.pow(-1.1)
    p /= p.sum()
    c = (p * M).floor().long()
    for e in empty:
        c[e] = 0
    c[int(rank.argmin())] += M - int(c.sum())  # the top expert takes the remainder
    assert int(c.sum()) == M and int(c.min()) >= 0
    return c


def _schedule_counts(E, tj, rounds, seed, blocks=256):
    """Expert loads whose persistent fwd / dgrad schedule (tj n-tiles per m-tile)
    holds about `rounds` rounds of `blocks` slots: a quarter of the experts thin (1-64
    rows, their tiles two per slot), eight empty, the rest full m-tiles plus a partial
    one of 65-256 rows."""
    g = torch.Generator().manual_seed(seed)
    nthin = E // 4
    target = int((rounds - 0.5) * blocks)
    mtiles = max((target - nthin * ((tj + 1) // 2)) // tj, E - nthin - 8)
    counts = torch.zeros(E, dtype=torch.long)
    counts[:nthin] = torch.randint(1, 65, (nthin,), generator=g)
    rest = list(range(nthin + 8, E))
    mt = torch.ones(len(rest), dtype=torch.long)
    if mtiles > len(rest):
        share = torch.multinomial(torch.ones(len(rest)), mtiles - len(rest), replacement=True,
                                  generator=g)
        mt += torch.bincount(share, minlength=len(rest))
    for i, e in enumerate(rest):
        counts[e] = (int(mt[i]) - 1) * 256 + int(torch.randint(65, 257, (1,), generator=g))
    return counts[torch.randperm(E, generator=g)]


@pytest.mark.parametrize("rounds,tj", [(1, 3), (7, 3), (12, 4), (14, 3), (6, 5)])
def test_grouped_matmul_cost_sorted_schedule_exact(rounds, tj):
    """Persistent fwd / dgrad launches of at most four n-tiles per m-tile and at most
    twelve rounds of schedule slots take a cost-sorted slot assignment within each XCD,
    computed by the kernel at start; longer launches and wider outputs keep the static
    order. Both sides of each limit, into NaN-filled outputs with small-integer
    operands: every row of every expert written, exactly. Thin experts (tiles two per
    slot), partial m-tiles and full ones mixed."""
    from torchturbo_amd import _lib

    torch.backends.cuda.matmul.allow_tf32 = False
    E, R = 96, 128
    counts = _schedule_counts(E, tj, rounds, seed=rounds * 10 + tj)
    M, J = int(counts.sum()), 256 * tj
    g = torch.Generator(device=DEV).manual_seed(tj)
    x = torch.randint(-2, 3, (M, R), generator=g, device=DEV).to(torch.bfloat16)
    w1 = torch.randint(-2, 3, (E, R, J), generator=g, device=DEV).to(torch.bfloat16)
    w2 = torch.randint(-2, 3, (E, J, R), generator=g, device=DEV).to(torch.bfloat16)
    y = torch.full((M, J), float("nan"), dtype=torch.bfloat16, device=DEV)
    dx = torch.full((M, J), float("nan"), dtype=torch.bfloat16, device=DEV)
    cnt = counts.to(DEV)
    bf = _lib.dtype_code(torch.bfloat16)
    # fwd: y = x w1 (K = R, N = J); dgrad: dx = x w2^T (K = J, N = R): J-wide outputs
    _lib.call("tt_gmm_fwd", _lib.ptr(x), _lib.ptr(w1), bf, M, R, J, E, 0, _lib.ptr(cnt),
              _lib.ptr(y), _lib.stream())
    _lib.call("tt_gmm_dgrad", _lib.ptr(x), _lib.ptr(w2), bf, M, J, R, E, 0, _lib.ptr(cnt),
              _lib.ptr(dx), _lib.stream())
    torch.cuda.synchronize()
    s0 = 0
    for e, c in enumerate(counts.tolist()):
        xe = x[s0:s0 + c].float()
        assert torch.equal(y[s0:s0 + c], (xe @ w1[e].float()).to(torch.bfloat16)), (e, c)
        assert torch.equal(dx[s0:s0 + c], (xe @ w2[e].float().t()).to(torch.bfloat16)), (e, c)
        s0 += c


# Shapes of the Qwen3-30B-A3B layer's two GEMMs (fc1: K 2048 -> N 1536, fc2: K 768 ->
# N 2048), tens of thousands of rows, Zipf loads with empty experts. Each launch has far
@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize("E,K,N", [(256, 512, 1536), (96, 320, 768), (40, 256, 1000), (24, 96, 200)])
def test_grouped_matmul_thin_experts_exact(trans_b, E, K, N):
    """Many experts of at most 64 rows (their output tiles are taken two per schedule
    slot by the persistent fwd / dgrad kernel, an odd number of column tiles leaving
    a slot with one) mixed with larger experts, some of whose last tiles are thin too,
    into NaN-filled outputs with small-integer operands: every row exact, in blocks
    that walk thin and full tiles in turn."""
    from torchturbo_amd import _lib

    torch.backends.cuda.matmul.allow_tf32 = False
    g = torch.Generator().manual_seed(E + K + N)
    small = torch.randint(1, 65, (E,), generator=g)
    big = torch.randint(65, 900, (E,), generator=g)
    counts = torch.where(torch.rand(E, generator=g) < 0.6, small, big)
    counts[0] = 0
    counts[1] = 64
    counts[2] = 65
    counts[3] = 256 + 64
    M = int(counts.sum())
    dtype = torch.bfloat16
    x = torch.randint(-2, 3, (M, K), generator=g).to(dtype).to(DEV)
    dy = torch.randint(-2, 3, (M, N), generator=g).to(dtype).to(DEV)
    wshape = (E, N, K) if trans_b else (E, K, N)
    w = torch.randint(-2, 3, wshape, generator=g).to(dtype).to(DEV)
    cnt = counts.to(DEV)
    args = (_lib.dtype_code(dtype), M, K, N, E, int(trans_b), _lib.ptr(cnt))
    for rep in range(2):  # the second call into outputs holding the first call's results
        y = torch.full((M, N), float("nan"), dtype=dtype, device=DEV)
        dx = torch.full((M, K), float("nan"), dtype=dtype, device=DEV)
        _lib.call("tt_gmm_fwd", _lib.ptr(x), _lib.ptr(w), *args, _lib.ptr(y), _lib.stream())
        _lib.call("tt_gmm_dgrad", _lib.ptr(dy), _lib.ptr(w), *args, _lib.ptr(dx), _lib.stream())
        torch.cuda.synchronize()
        wf = w.float()
        s0 = 0
        for e, c in enumerate(counts.tolist()):
            we = wf[e].t() if trans_b else wf[e]  # [K, N]
            assert torch.equal(y[s0:s0 + c], (x[s0:s0 + c].float() @ we).to(dtype)), (rep, e, c)
            assert torch.equal(dx[s0:s0 + c], (dy[s0:s0 + c].float() @ we.t()).to(dtype)), (rep, e, c)
            s0 += c


# more 256x256 output tiles than the GPU has compute units, so every persistent block
# walks many tiles (tile switch, cross-tile prefetch, XCD remap); mean expert loads above
# 512 rows take the four-stage weight-gradient kernel, at most 512 the persistent
# weight-gradient kernel with its ticket queues (many tickets per block).
MANY_TILES = [
    (torch.bfloat16, False, 64, 65536, 2048, 1536),
    (torch.bfloat16, True, 64, 65536, 2048, 1536),
    (torch.bfloat16, False, 64, 65536, 768, 2048),
    (torch.bfloat16, True, 128, 32768, 768, 2048),
    (torch.bfloat16, False, 128, 32768, 2048, 1536),
    (torch.float16, False, 128, 49152, 2048, 1536),
    (torch.bfloat16, False, 64, 40000, 2000, 1000),  # reduction tails: K, N not multiples of 64
]


@pytest.mark.parametrize("dtype,trans_b,E,M,K,N", MANY_TILES,
                         ids=lambda v: str(v).replace("torch.", ""))
def test_grouped_matmul_many_tiles(hip_ops, dtype, trans_b, E, M, K, N):
    """fwd, dgrad and wgrad against per-expert fp32 products (torch, same device)."""
    torch.backends.cuda.matmul.allow_tf32 = False
    counts = _zipf_counts(E, M, seed=E + K + N)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    slots = int(sum((int(c) + 255) // 256 for c in counts)) * ((N + 255) // 256)
    assert slots > 2 * cus, (slots, cus)  # several output tiles per persistent block
    g = torch.Generator(device=DEV).manual_seed(7)
    x = torch.randn(M, K, generator=g, device=DEV).to(dtype).requires_grad_()
    wshape = (E, N, K) if trans_b else (E, K, N)
    w = (torch.randn(*wshape, generator=g, device=DEV) * 0.05).to(dtype).requires_grad_()
    dy = torch.randn(M, N, generator=g, device=DEV).to(dtype)
    y = hip_ops.grouped_matmul(x, w, counts.to(DEV), trans_b=trans_b)
    y.backward(dy)
    xs = torch.split(x.detach().float(), counts.tolist())
    ds = torch.split(dy.float(), counts.tolist())
    wf = w.detach().float()
    yr, dxr, dwr = [], [], torch.zeros(wshape, device=DEV)
    for e in range(E):
        we = wf[e].t() if trans_b else wf[e]  # [K, N]
        yr.append(xs[e] @ we)
        dxr.append(ds[e] @ we.t())
        dwe = xs[e].t() @ ds[e]  # [K, N]
        dwr[e] = dwe.t() if trans_b else dwe
    for a, b, name in ((y, torch.cat(yr), "y"), (x.grad, torch.cat(dxr), "dx"), (w.grad, dwr, "dw")):
        mx, mean = rel_errors(a.float(), b)
        assert mx <= 1e-2 and mean <= 2e-3, f"{name}: {mx:.3e} {mean:.3e}"
    for e in (counts == 0).nonzero().flatten().tolist():
        assert torch.count_nonzero(w.grad[e]) == 0


@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize("E,K,N", [(64, 1024, 768), (13, 1024, 768), (13, 768, 768),
                                   (16, 2048, 1024), (13, 2048, 16384)])
def test_grouped_matmul_long_wgrad_integer_exact(hip_ops, trans_b, E, K, N):
    """Weight gradients with long expert reductions (mean load above 512 rows) on
    small-integer operands, so every sum is exact in fp32 and dW is the exact product
    rounded once. Zipf loads with empty experts, a one-row expert and experts shorter
    than three 32-deep k-tiles. Below 512 output tiles per expert the four-stage kernel
    takes them (one output tile per block, experts in the longest-first order of the
    launch's ranking): with a 4 x 3 or 8 x 4 tile grid every expert's tiles go to one
    pair of XCDs (at E = 13, not a multiple of 8, the blocks of ranks past the last
    expert exit); a 3 x 3 grid (no even side) takes the all-XCD mapping. An 8 x 64 grid
    takes the persistent kernel, whose longest reduction here runs to 91 64-deep
    k-tiles."""
    torch.backends.cuda.matmul.allow_tf32 = False
    counts = _zipf_counts(E, E * 1024, seed=5, empty=(3, 7) if E < 20 else (3, 17, 40))
    counts[11], counts[12] = 1, 70  # below three k-tiles
    counts[int(counts.argmax())] -= 71
    M = int(counts.sum())
    from torchturbo_amd import _lib

    tiles = -(-K // 256) * -(-N // 256)
    assert _lib.load().tt_gmm_wgrad_persistent(_lib.TT_BF16, M, K, N, E, int(trans_b)) == (tiles >= 512)
    g = torch.Generator(device=DEV).manual_seed(3)
    x = torch.randint(-3, 4, (M, K), generator=g, device=DEV).to(torch.bfloat16)
    wshape = (E, N, K) if trans_b else (E, K, N)
    w = torch.randint(-3, 4, wshape, generator=g, device=DEV).to(torch.bfloat16).requires_grad_()
    dy = torch.randint(-3, 4, (M, N), generator=g, device=DEV).to(torch.bfloat16)
    for _ in range(2):  # twice: nothing carries over between launches
        w.grad = None
        y = hip_ops.grouped_matmul(x, w, counts.to(DEV), trans_b=trans_b)
        y.backward(dy)
        xs = torch.split(x.float(), counts.tolist())
        ds = torch.split(dy.float(), counts.tolist())
        for e in range(E):
            dwe = xs[e].t() @ ds[e]  # [K, N], exact (integer sums below 2^24)
            ref = (dwe.t() if trans_b else dwe).to(torch.bfloat16)
            assert torch.equal(w.grad[e], ref), (e, int(counts[e]))


def test_grouped_matmul_wgrad_ranking_many_experts_exact(hip_ops):
    """The one-tile-per-block weight gradient takes experts longest first from a ranking
    computed once per launch (one thread per expert, a block per 256 experts). 300
    experts: a run of 80 equal loads (ranked by id), empty and one-row experts and one
    long expert, small-integer operands so dW is exact. A rank written twice or not at
    all would leave an expert's gradient unwritten or written from another's rows."""
    from torchturbo_amd import _lib

    torch.backends.cuda.matmul.allow_tf32 = False
    E, K, N = 300, 256, 512
    counts = torch.full((E,), 720, dtype=torch.int64)
    counts[::7] = 0
    counts[5::11] = 1
    counts[100:180] = 900
    counts[299] = 5000
    M = int(counts.sum())
    assert M > 512 * E
    assert _lib.load().tt_gmm_wgrad_persistent(_lib.TT_BF16, M, K, N, E, 0) == 0
    g = torch.Generator(device=DEV).manual_seed(11)
    x = torch.randint(-3, 4, (M, K), generator=g, device=DEV).to(torch.bfloat16)
    w = torch.randint(-3, 4, (E, K, N), generator=g, device=DEV).to(torch.bfloat16)
    w.requires_grad_()
    dy = torch.randint(-3, 4, (M, N), generator=g, device=DEV).to(torch.bfloat16)
    xs = torch.split(x.float(), counts.tolist())
    ds = torch.split(dy.float(), counts.tolist())
    ref = torch.stack([(a.t() @ b).to(torch.bfloat16) for a, b in zip(xs, ds)])
    for _ in range(2):  # twice: the second launch ranks into another slot
        w.grad = None
        y = hip_ops.grouped_matmul(x, w, counts.to(DEV))
        y.backward(dy)
        assert torch.equal(w.grad, ref)


# ---------------------------------------------------------------------------
# FP8 block-scaled grouped GEMM
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("counts,K,N", [([0, 130, 7, 256], 256, 384), ([64, 64], 512, 256),
                                         ([5, 0, 300, 129], 208, 272), ([128, 1, 90], 96, 640)])
def test_grouped_matmul_fp8(hip_ops, counts, K, N):
    g = torch.Generator().manual_seed(K + N)
    E, M = len(counts), sum(counts)
    master = torch.randn(E, N, K, generator=g) * 0.02
    q, s = o_fp8.quantize_experts(master)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    dy = torch.randn(M, N, generator=g).to(torch.bfloat16)
    deq = o_fp8.dequantize_experts(q, s)
    xr = x.double().requires_grad_()
    wr = deq.double().requires_grad_()
    yr = o_gmm.grouped_matmul(xr, wr, counts, trans_b=True)
    yr.backward(dy.double())
    xd = x.to(DEV).requires_grad_()
    md = deq.to(DEV).requires_grad_()
    y = hip_ops.grouped_matmul_fp8(xd, q.to(DEV), s.to(DEV), counts, master=md)
    y.backward(dy.to(DEV))
    for a, b, name in ((y, yr, "y"), (xd.grad, xr.grad, "dx"), (md.grad, wr.grad, "dw")):
        mx, mean = rel_errors(a.cpu(), b)
        assert mx <= 1e-2 and mean <= 2e-3, f"{name}: {mx:.3e} {mean:.3e}"


def test_fp8_dequant_exact_through_gemm(hip_ops):
    """x = unit rows selects single weight columns: y equals the dequantized weight bit-exactly."""
    E, N, K = 2, 256, 256
    g = torch.Generator().manual_seed(1)
    master = torch.randn(E, N, K, generator=g) * 0.3
    q, s = o_fp8.quantize_experts(master)
    deq = o_fp8.dequantize_experts(q, s)
    x = torch.eye(K).repeat(E, 1).to(torch.bfloat16)  # [E*K, K]
    y = hip_ops.grouped_matmul_fp8(x.to(DEV), q.to(DEV), s.to(DEV), [K] * E)
    expect = torch.cat([deq[e].t() for e in range(E)])  # row k of expert e = W[:, k]
    assert torch.equal(y.cpu(), expect)


def test_fp8_dequant_exact_through_dgrad(hip_ops):
    """dy = identity rows per expert: dx = dy @ W_deq returns the dequantized weight rows
    bit-exactly (each output is one product with 1.0 plus exact zeros); covers the
    N-major (transposed) e4m3 operand with partial 512-column tiles and partial
    scale blocks."""
    E, N, K = 3, 384, 320
    g = torch.Generator().manual_seed(2)
    master = torch.randn(E, N, K, generator=g) * 0.3
    q, s = o_fp8.quantize_experts(master)
    deq = o_fp8.dequantize_experts(q, s)
    x = torch.randn(E * N, K, generator=g).to(torch.bfloat16).to(DEV).requires_grad_()
    y = hip_ops.grouped_matmul_fp8(x, q.to(DEV), s.to(DEV), [N] * E)
    y.backward(torch.eye(N).repeat(E, 1).to(torch.bfloat16).to(DEV))
    assert torch.equal(x.grad.cpu(), deq.reshape(E * N, K))


def test_grouped_matmul_fp8_many_tiles(hip_ops):
    """More output tiles than compute units (each persistent block walks several
    tiles), skewed loads with empty experts; fp32 reference of the dequantized weights."""
    E, K, N = 64, 512, 1024
    g = torch.Generator().manual_seed(5)
    counts = [int(c) for c in torch.randint(0, 600, (E,), generator=g)]
    counts[3] = counts[17] = 0
    M = sum(counts)
    master = torch.randn(E, N, K, generator=g) * 0.02
    q, s = o_fp8.quantize_experts(master)
    deq = o_fp8.dequantize_experts(q, s).to(DEV)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV).requires_grad_()
    dy = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV)
    mw = deq.clone().requires_grad_()  # bf16 master weights [E, N, K]
    y = hip_ops.grouped_matmul_fp8(x, q.to(DEV), s.to(DEV), counts, master=mw)
    y.backward(dy)
    xs = torch.split(x.detach().float(), counts)
    ds = torch.split(dy.float(), counts)
    yr = torch.cat([xs[e] @ deq[e].float().t() for e in range(E)])
    dxr = torch.cat([ds[e] @ deq[e].float() for e in range(E)])
    # master-weight gradient dW[e] = dy_e^T @ x_e ([N, K]); empty experts exactly zero
    dwr = torch.stack([ds[e].t() @ xs[e] for e in range(E)])
    for a, b, name in ((y, yr, "y"), (x.grad, dxr, "dx"), (mw.grad, dwr, "d_master")):
        mx, mean = rel_errors(a.float().cpu(), b.cpu())
        assert mx <= 1e-2 and mean <= 2e-3, f"{name}: {mx:.3e} {mean:.3e}"
    for e in (3, 17):
        assert torch.count_nonzero(mw.grad[e]) == 0, e
