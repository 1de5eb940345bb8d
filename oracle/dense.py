"""Per-token dense loop for tiny MoE layers (CPU oracle).

Restates the loop of ``tests/models/test_moe_probability_weighting.py:134-165``
for the softmax / sigmoid routers: for every token and each of its k experts
compute ``(swiglu(x W1_e) * p) W2_e`` and sum the k contributions. It is
independent of the packed layout, so it checks the permutation,
grouped-matmul and unpermutation composition as a whole.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def dense_moe(hidden, ids, topk_probs, w1, w2):
    """hidden [T, H]; ids [T, k]; topk_probs [T, k]; w1 [E, H, 2F]; w2 [E, F, H]."""
    rows = []
    for t in range(hidden.shape[0]):
        parts = []
        for j in range(ids.shape[1]):
            e = int(ids[t, j])
            p = topk_probs[t, j].unsqueeze(0)
            gate, up = (hidden[t] @ w1[e]).chunk(2, dim=-1)
            act = (F.silu(gate) * up)
            act = (act * p).to(act.dtype)
            parts.append(act @ w2[e])
        rows.append(torch.stack(parts).sum(0))
    return torch.stack(rows).to(hidden.dtype)
