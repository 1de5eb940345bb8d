"""Packed-row order of the MoE permutation in numpy (CPU oracle, integer work).

The contract (``src/torchturbo/ops/moe.py:10-46``) fixes the packed order:
expert id ascending, then source token ascending. For top-k ids ``ids[T, k]``
(distinct per token) this is a stable sort of the T*k assignments by expert
id when they are listed token-major, which is what
``np.argsort(kind="stable")`` computes. ``brute_force`` restates it with
plain loops over (expert, token) for tiny inputs.

Pinned by: ``brute_force`` on tiny inputs and the literal row maps of
``tests/ops/test_moe_permutation_contract.py:72-84,307-370``.
"""

from __future__ import annotations

import numpy as np


def route_index(ids: np.ndarray, num_experts: int):
    """ids [T, k] int -> (row_indices [T, k] int32, token_of_row [T*k] int32,
    counts [E] int64, offsets [E+1] int64)."""
    ids = np.asarray(ids, dtype=np.int64)
    num_tokens, topk = ids.shape
    flat = ids.reshape(-1)
    order = np.argsort(flat, kind="stable")  # packed row -> flat slot
    rows = np.empty(flat.size, dtype=np.int32)
    rows[order] = np.arange(flat.size, dtype=np.int32)
    counts = np.bincount(flat, minlength=num_experts).astype(np.int64)
    offsets = np.zeros(num_experts + 1, dtype=np.int64)
    np.cumsum(counts, out=offsets[1:])
    token_of_row = (order // max(topk, 1)).astype(np.int32)
    return rows.reshape(num_tokens, topk), token_of_row, counts, offsets


def brute_force(ids, num_experts: int):
    """Same outputs by enumerating (expert, token) pairs in order."""
    ids = [list(map(int, r)) for r in ids]
    num_tokens = len(ids)
    topk = len(ids[0]) if ids else 0
    rows = [[-1] * topk for _ in range(num_tokens)]
    token_of_row = []
    counts = [0] * num_experts
    row = 0
    for e in range(num_experts):
        for t in range(num_tokens):
            for j in range(topk):
                if ids[t][j] == e:
                    rows[t][j] = row
                    token_of_row.append(t)
                    counts[e] += 1
                    row += 1
    offsets = [0]
    for c in counts:
        offsets.append(offsets[-1] + c)
    return (np.array(rows, dtype=np.int32).reshape(num_tokens, topk),
            np.array(token_of_row, dtype=np.int32), np.array(counts), np.array(offsets))
