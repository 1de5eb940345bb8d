"""``tt_route_index_noalloc`` (fixed device scratch, no workspace) against
``tt_route_index`` (caller workspace), called through the C-ABI: row map,
packed-row tokens, packed probs, counts and the rejected-slot count agree
bit for bit, on two calls in a row (the second smaller, so it runs over the
first call's leftovers in the shared scratch), and problems beyond the fixed
scratch are refused with an error instead of running."""

from __future__ import annotations

import pytest
import torch

from torchturbo_amd import _lib as L

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ids(T, E, k, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    ids = torch.rand(T, E, generator=g, device=DEV).topk(k, dim=1).indices
    ids[7 % T, 0] = E                # out of range: rejected
    ids[11 % T, k - 1] = ids[11 % T, 0]  # repeated: rejected
    return ids.contiguous()


def _outputs(T, E, k, probs):
    rows = torch.full((T, k), -9, dtype=torch.int32, device=DEV)
    tor = torch.full((T * k,), -9, dtype=torch.int32, device=DEV)
    pp = torch.zeros(T * k, dtype=probs.dtype, device=DEV)
    counts = torch.full((E,), -9, dtype=torch.int64, device=DEV)
    return rows, tor, pp, counts


def _with_workspace(ids, E, probs):
    T, k = ids.shape
    rows, tor, pp, counts = _outputs(T, E, k, probs)
    nbytes = L.route_index_workspace(T, E)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    L.call("tt_route_index", L.ptr(ids), T, k, E, L.ptr(probs), L.dtype_code(probs.dtype),
           L.ptr(rows), L.ptr(tor), L.ptr(pp), L.ptr(counts), L.ptr(ws), nbytes, L.stream())
    off = L.route_index_rejected_offset(T, E)
    rejected = ws[off:off + 4].view(torch.int32).clone()
    return rows, tor, pp, counts, rejected


def _no_alloc(ids, E, probs):
    T, k = ids.shape
    rows, tor, pp, counts = _outputs(T, E, k, probs)
    rejected = torch.full((1,), -9, dtype=torch.int32, device=DEV)
    L.call("tt_route_index_noalloc", L.ptr(ids), T, k, E, L.ptr(probs),
           L.dtype_code(probs.dtype), L.ptr(rows), L.ptr(tor), L.ptr(pp), L.ptr(counts),
           L.ptr(rejected), L.stream())
    return rows, tor, pp, counts, rejected


@pytest.mark.parametrize("first,second", [((16384, 128, 8), (3000, 64, 6)),
                                          ((4096, 256, 8), (517, 33, 3))])
def test_route_index_noalloc_matches_workspace_entry(first, second):
    for i, (T, E, k) in enumerate((first, second)):
        ids = _ids(T, E, k, seed=T + E)
        probs = torch.rand(T, E, device=DEV)
        ref = _with_workspace(ids, E, probs)
        got = _no_alloc(ids, E, probs)
        torch.cuda.synchronize()
        n = int(ref[3].sum())
        assert int(ref[4]) == 2 and n == T * k - 2, (i, int(ref[4]), n)
        for name, a, b in zip(("rows", "token_of_row", "packed_probs", "counts", "rejected"),
                              got, ref):
            if name in ("token_of_row", "packed_probs"):
                a, b = a[:n], b[:n]  # rows past the accepted ones are never written
            assert torch.equal(a, b), (i, name)


def test_route_index_noalloc_without_rejected_output_and_limits():
    T, E, k = 2048, 64, 4
    ids = _ids(T, E, k, seed=3)
    probs = torch.rand(T, E, device=DEV, dtype=torch.bfloat16)
    ref = _with_workspace(ids, E, probs)
    rows, tor, pp, counts = _outputs(T, E, k, probs)
    L.call("tt_route_index_noalloc", L.ptr(ids), T, k, E, L.ptr(probs),
           L.dtype_code(probs.dtype), L.ptr(rows), L.ptr(tor), L.ptr(pp), L.ptr(counts), None,
           L.stream())
    torch.cuda.synchronize()
    assert torch.equal(rows, ref[0]) and torch.equal(counts, ref[3])
    # 600k tokens over 128 experts need about 1.2 MiB of histograms: refused, nothing runs
    big = 600_000
    assert L.route_index_workspace(big, 128) > (1 << 20)
    with pytest.raises(ValueError, match="fixed"):
        L.call("tt_route_index_noalloc", None, big, 8, 128, None, 0, None, None, None, None,
               None, L.stream())
