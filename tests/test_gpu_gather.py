"""Grouped GEMMs that gather their activation rows (GPU).

``tt_gmm_fwd_gather`` / ``tt_gmm_dgrad_gather`` read packed row r from row
``src_of_row[r]`` of an unpacked source, so a permutation and the GEMM after it
are one launch. They must equal the packed GEMMs (``tt_gmm_fwd`` /
``tt_gmm_dgrad``) on ``src[src_of_row]`` bit for bit: same operand values, same
reduction order. Cases: many tiles per persistent block (Qwen shapes), Zipf
loads with empty and one-row experts, duplicated and unused source rows, both
weight layouts, bf16 and f16.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _loads(E, M, seed):
    g = torch.Generator().manual_seed(seed)
    rank = torch.randperm(E, generator=g).double() + 1.0
    c = (rank.pow(-1.1) / rank.pow(-1.1).sum() * M).floor().long()
    c[min(3, E - 1)] = 0
    c[min(4, E - 1)] = 1
    c[int(rank.argmin())] += M - int(c.sum())
    assert int(c.sum()) == M and int(c.min()) >= 0
    return c


# dtype, trans_b, E, M (packed rows), T (source rows), K, N
CASES = [
    (torch.bfloat16, False, 128, 65536, 8192, 2048, 1536),
    (torch.bfloat16, True, 64, 32768, 4096, 768, 2048),
    (torch.float16, False, 13, 9000, 2000, 512, 768),
    (torch.bfloat16, False, 5, 700, 60, 128, 192),
]


@pytest.mark.parametrize("dtype,trans_b,E,M,T,K,N", CASES,
                         ids=lambda v: str(v).replace("torch.", ""))
def test_gathered_rows_equal_the_packed_gemm(dtype, trans_b, E, M, T, K, N):
    from torchturbo_amd import _lib

    counts = _loads(E, M, seed=E + K)
    g = torch.Generator(device=DEV).manual_seed(11)
    xs = torch.randn(T, K, generator=g, device=DEV).to(dtype)
    dys = torch.randn(T, N, generator=g, device=DEV).to(dtype)
    rows = torch.randint(0, T, (M,), generator=g, device=DEV, dtype=torch.int32)
    wshape = (E, N, K) if trans_b else (E, K, N)
    w = (torch.randn(*wshape, generator=g, device=DEV) * 0.05).to(dtype)
    cnt = counts.to(DEV)
    args = (_lib.dtype_code(dtype), M, K, N, E, int(trans_b), _lib.ptr(cnt))
    st = _lib.stream()
    y_p = torch.empty(M, N, dtype=dtype, device=DEV)
    dx_p = torch.empty(M, K, dtype=dtype, device=DEV)
    x_packed, dy_packed = xs[rows.long()], dys[rows.long()]
    _lib.call("tt_gmm_fwd", _lib.ptr(x_packed), _lib.ptr(w), *args, _lib.ptr(y_p), st)
    _lib.call("tt_gmm_dgrad", _lib.ptr(dy_packed), _lib.ptr(w), *args, _lib.ptr(dx_p), st)
    for _ in range(2):  # twice into NaN-filled outputs: every row written, nothing carried over
        y_g = torch.full((M, N), float("nan"), dtype=dtype, device=DEV)
        dx_g = torch.full((M, K), float("nan"), dtype=dtype, device=DEV)
        _lib.call("tt_gmm_fwd_gather", _lib.ptr(xs), T, _lib.ptr(rows), _lib.ptr(w), *args,
                  _lib.ptr(y_g), st)
        _lib.call("tt_gmm_dgrad_gather", _lib.ptr(dys), T, _lib.ptr(rows), _lib.ptr(w), *args,
                  _lib.ptr(dx_g), st)
        torch.cuda.synchronize()
        assert torch.equal(y_g, y_p)
        assert torch.equal(dx_g, dx_p)


def test_gather_rejects_reductions_it_does_not_cover():
    """Reductions of 64 or fewer, or not a multiple of 64, take kernels without a
    gathered path: the call fails before any launch."""
    from torchturbo_amd import _lib

    counts = torch.tensor([3, 5], device=DEV)
    xs = torch.zeros(8, 96, dtype=torch.bfloat16, device=DEV)
    rows = torch.zeros(8, dtype=torch.int32, device=DEV)
    w = torch.zeros(2, 96, 64, dtype=torch.bfloat16, device=DEV)
    y = torch.empty(8, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="multiple of 64"):
        _lib.call("tt_gmm_fwd_gather", _lib.ptr(xs), 8, _lib.ptr(rows), _lib.ptr(w), 1, 8, 96, 64,
                  2, 0, _lib.ptr(counts), _lib.ptr(y), _lib.stream())


# dtype, trans_b, gathered operand, E, M, T, K, N (more than 512 rows per expert on average)
WGRAD_CASES = [
    (torch.bfloat16, False, "x", 64, 65536, 8192, 2048, 1536),
    (torch.bfloat16, False, "dy", 64, 65536, 8192, 768, 2048),
    (torch.bfloat16, True, "x", 16, 12000, 3000, 512, 768),
    (torch.bfloat16, True, "dy", 16, 12000, 3000, 512, 768),
    (torch.float16, False, "dy", 13, 9000, 2000, 256, 512),
]


@pytest.mark.parametrize("dtype,trans_b,which,E,M,T,K,N", WGRAD_CASES,
                         ids=lambda v: str(v).replace("torch.", ""))
def test_gathered_wgrad_equals_the_packed_wgrad(dtype, trans_b, which, E, M, T, K, N):
    """tt_gmm_wgrad_gather with the rows of x or of dy gathered equals tt_gmm_wgrad on the
    gathered rows bit for bit (Zipf loads with empty and one-row experts, so some
    reductions end inside a k-tile and some experts have none)."""
    from torchturbo_amd import _lib

    counts = _loads(E, M, seed=3 * E + N)
    g = torch.Generator(device=DEV).manual_seed(5)
    rows = torch.randint(0, T, (M,), generator=g, device=DEV, dtype=torch.int32)
    if which == "x":
        src = torch.randn(T, K, generator=g, device=DEV).to(dtype)
        other = torch.randn(M, N, generator=g, device=DEV).to(dtype)
        x_p, dy_p = src[rows.long()], other
    else:
        src = torch.randn(T, N, generator=g, device=DEV).to(dtype)
        other = torch.randn(M, K, generator=g, device=DEV).to(dtype)
        x_p, dy_p = other, src[rows.long()]
    wshape = (E, N, K) if trans_b else (E, K, N)
    cnt = counts.to(DEV)
    tail = (_lib.dtype_code(dtype), M, K, N, E, int(trans_b), _lib.ptr(cnt))
    st = _lib.stream()
    dw_p = torch.empty(wshape, dtype=dtype, device=DEV)
    _lib.call("tt_gmm_wgrad", _lib.ptr(x_p), _lib.ptr(dy_p), *tail, _lib.ptr(dw_p), st)
    for _ in range(2):
        dw_g = torch.full(wshape, float("nan"), dtype=dtype, device=DEV)
        if which == "x":
            _lib.call("tt_gmm_wgrad_gather", _lib.ptr(src), T, _lib.ptr(rows), _lib.ptr(other),
                      0, None, *tail, _lib.ptr(dw_g), st)
        else:
            _lib.call("tt_gmm_wgrad_gather", _lib.ptr(other), 0, None, _lib.ptr(src), T,
                      _lib.ptr(rows), *tail, _lib.ptr(dw_g), st)
        torch.cuda.synchronize()
        assert torch.equal(dw_g, dw_p)


def test_gathered_rows_out_of_range_read_zeros():
    """Row-map entries outside [0, src_rows) (-1, src_rows, 2^30) read rows of
    zeros in every gathering GEMM: the results equal the packed GEMMs with zero
    rows there (the header's contract), not a wrapped-around source row."""
    from torchturbo_amd import _lib

    dtype, E, M, T, K, N = torch.bfloat16, 13, 9000, 2000, 512, 768
    counts = _loads(E, M, seed=77)
    g = torch.Generator(device=DEV).manual_seed(3)
    rows = torch.randint(0, T, (M,), generator=g, device=DEV, dtype=torch.int32)
    bad = torch.randperm(M, generator=g, device=DEV)[:M // 20]
    rows[bad[0::3]] = -1
    rows[bad[1::3]] = T
    rows[bad[2::3]] = 1 << 30
    inside = (rows >= 0) & (rows < T)
    eff = torch.where(inside, rows, torch.full_like(rows, T)).long()
    xs = torch.randn(T, K, generator=g, device=DEV).to(dtype)
    dys = torch.randn(T, N, generator=g, device=DEV).to(dtype)
    x_packed = torch.cat([xs, xs.new_zeros(1, K)])[eff]
    dy_packed = torch.cat([dys, dys.new_zeros(1, N)])[eff]
    w = (torch.randn(E, K, N, generator=g, device=DEV) * 0.05).to(dtype)
    cnt = counts.to(DEV)
    args = (_lib.dtype_code(dtype), M, K, N, E, 0, _lib.ptr(cnt))
    st = _lib.stream()
    y_p, y_g = (torch.empty(M, N, dtype=dtype, device=DEV) for _ in range(2))
    dx_p, dx_g = (torch.empty(M, K, dtype=dtype, device=DEV) for _ in range(2))
    _lib.call("tt_gmm_fwd", _lib.ptr(x_packed), _lib.ptr(w), *args, _lib.ptr(y_p), st)
    _lib.call("tt_gmm_dgrad", _lib.ptr(dy_packed), _lib.ptr(w), *args, _lib.ptr(dx_p), st)
    _lib.call("tt_gmm_fwd_gather", _lib.ptr(xs), T, _lib.ptr(rows), _lib.ptr(w), *args,
              _lib.ptr(y_g), st)
    _lib.call("tt_gmm_dgrad_gather", _lib.ptr(dys), T, _lib.ptr(rows), _lib.ptr(w), *args,
              _lib.ptr(dx_g), st)
    torch.cuda.synchronize()
    assert torch.equal(y_g, y_p)
    assert torch.equal(dx_g, dx_p)
    assert not y_g[~inside].any()
    other_dy = torch.randn(M, N, generator=g, device=DEV).to(dtype)
    other_x = torch.randn(M, K, generator=g, device=DEV).to(dtype)
    for which in ("x", "dy"):
        xp, dyp = (x_packed, other_dy) if which == "x" else (other_x, dy_packed)
        dw_p = torch.empty(E, K, N, dtype=dtype, device=DEV)
        dw_g = torch.full((E, K, N), float("nan"), dtype=dtype, device=DEV)
        _lib.call("tt_gmm_wgrad", _lib.ptr(xp), _lib.ptr(dyp), *args, _lib.ptr(dw_p), st)
        if which == "x":
            _lib.call("tt_gmm_wgrad_gather", _lib.ptr(xs), T, _lib.ptr(rows), _lib.ptr(other_dy),
                      0, None, *args, _lib.ptr(dw_g), st)
        else:
            _lib.call("tt_gmm_wgrad_gather", _lib.ptr(other_x), 0, None, _lib.ptr(dys), T,
                      _lib.ptr(rows), *args, _lib.ptr(dw_g), st)
        torch.cuda.synchronize()
        assert torch.equal(dw_g, dw_p), which


def test_gathered_wgrad_rejects_short_reductions():
    """At most 512 rows per expert on average the persistent weight-gradient kernel
    runs, which has no gathered path: the call fails before any launch."""
    from torchturbo_amd import _lib

    counts = torch.tensor([300, 200], device=DEV)
    src = torch.zeros(10, 128, dtype=torch.bfloat16, device=DEV)
    rows = torch.zeros(500, dtype=torch.int32, device=DEV)
    dy = torch.zeros(500, 128, dtype=torch.bfloat16, device=DEV)
    dw = torch.empty(2, 128, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="512 rows"):
        _lib.call("tt_gmm_wgrad_gather", _lib.ptr(src), 10, _lib.ptr(rows), _lib.ptr(dy), 0, None,
                  1, 500, 128, 128, 2, 0, _lib.ptr(counts), _lib.ptr(dw), _lib.stream())


def _run_layer(layer, hidden, logits, grad):
    for p in layer.parameters():
        p.grad = None
    hd = hidden.clone().requires_grad_()
    ld = logits.clone().requires_grad_()
    out = layer.forward_with_logits(hd, ld)
    out.backward(grad)
    return (out.detach(), hd.grad, ld.grad, layer.experts.weight1.grad.clone(),
            layer.experts.weight2.grad.clone(), layer.token_dispatcher.tokens_per_expert.clone())


@pytest.mark.parametrize("tokens,hidden,ffn,experts,topk,logits", [
    (4096, 512, 256, 16, 4, "zipf"),
    (4096, 1024, 384, 8, 2, "normal"),
])
def test_layer_gathering_experts_equal_the_dispatched_path(process_ops, monkeypatch, tokens,
                                                           hidden, ffn, experts, topk, logits):
    """MoELayer with the permutation and unpermutation folded into the GEMMs (the
    default on one GPU when the shapes allow) gives the output, every gradient and the
    per-expert counts of the permute -> GroupedMLP -> unpermute path bit for bit."""
    from dataclasses import replace

    from tests.test_gpu_layer import build_layer
    from torchturbo_amd import configs as C
    from torchturbo_amd.dispatch import OpPolicy
    from torchturbo_amd.runtime import CudaRuntime

    process_ops(CudaRuntime(), OpPolicy.CUSTOM)
    w = replace(C.QWEN3, tokens=tokens, hidden=hidden, ffn=ffn, experts=experts, topk=topk,
                logits=logits)
    hidden_t = C.make_hidden(w).to(DEV)
    logits_t = C.make_logits(w).to(DEV)
    w1, w2 = C.make_weights(w)
    grad = C.make_grad(w).to(DEV)
    layer = build_layer(w, w1, w2)
    flat = hidden_t.view(-1, hidden)
    ids = logits_t.topk(topk, dim=1).indices
    monkeypatch.setenv("TORCHTURBO_AMD_FUSED_PERMUTE", "1")
    assert layer._gathering_experts(flat, ids)
    fused = _run_layer(layer, hidden_t, logits_t, grad)
    monkeypatch.setenv("TORCHTURBO_AMD_FUSED_PERMUTE", "0")
    assert not layer._gathering_experts(flat, ids)
    plain = _run_layer(layer, hidden_t, logits_t, grad)
    for a, b, name in zip(fused, plain, ("out", "d_hidden", "d_logits", "d_w1", "d_w2", "counts")):
        assert torch.equal(a, b), name


def test_gathering_experts_check_their_routing_input(process_ops):
    """The folded path runs the same input checks as the dispatched one: with checks on,
    an out-of-range expert id and a routing map that disagrees with the ids raise
    ValueError before any GEMM."""
    from torchturbo_amd import checks
    from torchturbo_amd.dispatch import OpPolicy
    from torchturbo_amd.moe import GroupedMLP, MoEConfig
    from torchturbo_amd.providers.hip import fused_experts
    from torchturbo_amd.runtime import CudaRuntime

    process_ops(CudaRuntime(), OpPolicy.CUSTOM)

    T, H, F, E, k = 2048, 256, 128, 4, 2  # 1024 rows per expert: the folded path's shapes
    cfg = MoEConfig(hidden_size=H, num_moe_experts=E, moe_ffn_hidden_size=F,
                    gated_linear_unit=True, activation_func=torch.nn.functional.silu,
                    moe_router_topk=k, params_dtype=torch.bfloat16)
    experts = GroupedMLP(E, False, cfg).to(DEV)
    with torch.no_grad():
        experts.weight1.normal_(0, 0.02)
        experts.weight2.normal_(0, 0.02)
    tokens = torch.randn(T, H, device=DEV).to(torch.bfloat16)
    assert fused_experts.eligible(tokens, experts.weight1, k, E)
    g = torch.Generator().manual_seed(1)
    ids = torch.rand(T, E, generator=g).topk(k, dim=1).indices
    rmap = torch.zeros(T, E, dtype=torch.bool).scatter(1, ids, True)
    probs = torch.rand(T, E).masked_fill(~rmap, 0.0)
    bad = ids.clone()
    bad[7, 1] = E
    other = ids.clone()
    other[3, 0] = [e for e in range(E) if e not in ids[3].tolist()][0]
    with checks.checking():
        with pytest.raises(ValueError, match="1 of 4096 slots"):
            fused_experts.grouped_mlp_tokens(experts, tokens, probs.to(DEV), rmap.to(DEV),
                                             bad.to(DEV))
        with pytest.raises(ValueError, match="disagree for 1 of 2048 tokens"):
            fused_experts.grouped_mlp_tokens(experts, tokens, probs.to(DEV), rmap.to(DEV),
                                             other.to(DEV))
        out, counts = fused_experts.grouped_mlp_tokens(experts, tokens, probs.to(DEV),
                                                       rmap.to(DEV), ids.to(DEV))
        assert out.shape == (T, H) and int(counts.sum()) == T * k
