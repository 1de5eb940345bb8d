"""Opt-in input checks (host logic, CPU): the routing-map / expert-id agreement
and the chunk-sort metadata checks raise ``ValueError`` where the reference's
native path raises (``ops/moe.py:62-65``, ``torch.split`` in
``native/moe_permutation.py:117-119``)."""

from __future__ import annotations

import pytest
import torch

from torchturbo_amd import checks
from torchturbo_amd.providers.hip.moe_permutation import _check_chunks, _check_map_matches_indices


def test_switch_and_context():
    saved = checks.enabled()
    with checks.checking(True):
        assert checks.enabled()
        with checks.checking(False):
            assert not checks.enabled()
        assert checks.enabled()
    assert checks.enabled() == saved


def test_map_and_indices_must_agree():
    ids = torch.tensor([[0, 2], [1, 3], [3, 0]])
    rmap = torch.zeros(3, 4, dtype=torch.bool).scatter(1, ids, True)
    _check_map_matches_indices(rmap, ids)
    _check_map_matches_indices(rmap[:0], ids[:0])
    with pytest.raises(ValueError, match="disagree for 1 of 3"):
        _check_map_matches_indices(rmap, torch.tensor([[0, 2], [1, 2], [3, 0]]))
    ragged = rmap.clone()
    ragged[1, 0] = True  # three experts selected for token 1
    with pytest.raises(ValueError, match="exactly its 2"):
        _check_map_matches_indices(ragged, ids)


def test_chunk_metadata():
    _check_chunks(10, torch.tensor([6, 0, 4]), torch.tensor([2, 0, 1]))
    _check_chunks(0, torch.tensor([], dtype=torch.long), torch.tensor([], dtype=torch.long))
    with pytest.raises(ValueError, match="sum to 9"):
        _check_chunks(10, torch.tensor([5, 4]), torch.tensor([1, 0]))
    with pytest.raises(ValueError, match="sum to 10"):
        _check_chunks(10, torch.tensor([12, -2]), torch.tensor([1, 0]))
    with pytest.raises(ValueError, match="permutation"):
        _check_chunks(10, torch.tensor([5, 5]), torch.tensor([1, 1]))
    with pytest.raises(ValueError, match="permutation"):
        _check_chunks(10, torch.tensor([5, 5]), torch.tensor([0, 2]))
