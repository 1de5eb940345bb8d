"""Pin the oracle with checks that do not restate its own formulas (CPU).

* routing index: numpy stable sort vs brute-force enumeration vs the torch
  restatement, on random tiny inputs (a dropped or swapped index fails);
* e4m3fn decode: all 256 codes vs the OCP E4M3 definition;
* grouped matmul: small-integer operands, exact in fp32, vs a float64
  triple loop;
* SwiGLU: closed forms (silu(0) = 0, silu(x) -> x for large x) and
  finite differences of the gradient;
* router: softmax-of-top-k equals renormalised full softmax (an identity),
  sigmoid probabilities sum to the scaling factor;
* unpermutation order: the sum of a token's rows is accumulated in ascending
  packed-row order in fp32 (a different order changes the fp32 result on a
  crafted input).
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import fp8 as o_fp8
from oracle import route_np
from oracle.native_providers import grouped_matmul as o_gmm
from oracle.native_providers import moe_permutation as o_perm
from oracle.native_providers import routing as o_route
from oracle.native_providers import swiglu as o_swiglu
from torchturbo_amd.dispatch import MoEPermutation


@pytest.mark.parametrize("seed", range(6))
def test_route_index_three_ways(seed):
    rng = np.random.default_rng(seed)
    T, E, k = int(rng.integers(1, 12)), int(rng.integers(2, 9)), 0
    k = int(rng.integers(1, min(E, 4) + 1))
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    a = route_np.route_index(ids, E)
    b = route_np.brute_force(ids, E)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
    rmap = torch.zeros(T, E, dtype=torch.bool)
    rmap.scatter_(1, torch.from_numpy(ids), True)
    perm = o_perm.permute(torch.arange(T, dtype=torch.float32)[:, None], rmap,
                          expert_indices=torch.from_numpy(ids))
    assert np.array_equal(perm.row_indices.numpy(), a[0])
    assert np.array_equal(perm.tokens[:, 0].numpy().astype(np.int32), a[1])


def test_e4m3fn_all_codes():
    codes = torch.arange(256, dtype=torch.uint8)
    vals = codes.view(torch.float8_e4m3fn).to(torch.float32).tolist()
    for c, v in zip(range(256), vals):
        ref = o_fp8.e4m3fn_decode(c)
        if math.isnan(ref):
            assert math.isnan(v), c
        else:
            assert v == ref, (c, v, ref)
    assert o_fp8.e4m3fn_decode(0x7E) == 448.0 and o_fp8.e4m3fn_decode(0x01) == 2.0 ** -9


def test_quantize_round_trip_error_bound():
    g = torch.Generator().manual_seed(0)
    w = torch.randn(256, 384, generator=g) * 0.02
    q, s = o_fp8.quantize_blockwise(w)
    deq = o_fp8.dequantize_weight(q, s).float()
    # e4m3 keeps 3 mantissa bits: relative error <= 2^-4 per element plus
    # the bf16 roundings of the scale and the result.
    rel = ((deq - w).abs() / w.abs().clamp_min(1e-6))
    big = w.abs() > 1e-3
    assert rel[big].max().item() < 0.08


def test_grouped_matmul_integer_exact():
    g = torch.Generator().manual_seed(1)
    counts = [3, 0, 5, 2]
    x = torch.randint(-4, 5, (10, 6), generator=g).float()
    w = torch.randint(-4, 5, (4, 6, 7), generator=g).float()
    y = o_gmm.grouped_matmul(x, w, counts)
    ref = torch.zeros(10, 7, dtype=torch.float64)
    start = 0
    for e, c in enumerate(counts):
        for r, j, kk in itertools.product(range(start, start + c), range(7), range(6)):
            ref[r, j] += float(x[r, kk]) * float(w[e, kk, j])
        start += c
    assert torch.equal(y.double(), ref)


def test_swiglu_closed_forms_and_fd_gradient():
    x = torch.tensor([[0.0, 30.0, -30.0, 2.0, 3.0, 1.0]])  # gate [0, 30, -30], up [2, 3, 1]
    out = o_swiglu.swiglu(x)
    assert out[0, 0].item() == 0.0
    assert abs(out[0, 1].item() - 90.0) < 1e-4
    assert abs(out[0, 2].item()) < 1e-9
    xd = torch.randn(4, 10, dtype=torch.float64, requires_grad=True)
    p = torch.rand(4, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda a, b: o_swiglu.swiglu_probs(a, b), (xd, p))


def test_router_identities():
    g = torch.Generator().manual_seed(2)
    logits = torch.randn(50, 16, generator=g, dtype=torch.float64)
    probs, _, ids = o_route.topk_softmax_with_capacity(logits, 4)
    full = logits.softmax(-1).gather(1, ids)
    torch.testing.assert_close(probs.gather(1, ids), full / full.sum(-1, keepdim=True))
    # ids are the 4 largest logits, descending
    assert torch.equal(ids, logits.argsort(-1, descending=True)[:, :4])
    probs, _, _ = o_route.topk_softmax_with_capacity(logits, 4, score_function="sigmoid",
                                                      scaling_factor=2.5)
    torch.testing.assert_close(probs.sum(-1), torch.full((50,), 2.5, dtype=torch.float64))


def test_unpermutation_sums_in_ascending_row_order():
    # fp32: 2^24 + 1 + 1 - 2^24 is 0 in ascending order and 2 if the +1s come
    # after the cancellation; rows given out of order in the slots.
    vals = torch.tensor([[2.0 ** 24], [1.0], [1.0], [-(2.0 ** 24)]])
    perm = MoEPermutation(vals, None, torch.tensor([[3, 1, 0, 2]], dtype=torch.int32),
                          torch.tensor([[3, 1, 0, 2]]))
    out = o_perm.unpermute(perm, torch.Size([1, 1]))
    assert out.item() == 0.0
    # the alternative order would give 2
    assert ((vals[0] + vals[3]) + vals[1] + vals[2]).item() == 2.0
