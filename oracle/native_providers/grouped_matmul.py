"""Native grouped matmul (CPU oracle).

Restates ``src/torchturbo/ops/providers/native/grouped_matmul.py:16-56``:
for each expert e with ``n_e`` rows starting at ``s_e``,
``Y[s_e:s_e+n_e] = X[s_e:s_e+n_e] @ W[e]`` (``W[e].T`` when ``trans_b``);
empty experts are skipped; ``[0, N]`` when every expert is empty. Backward is
PyTorch autograd of the same loop (dX_e = dY_e W_e^T, dW_e = X_e^T dY_e, zero
for empty experts; contract mirrored by
``src/torchturbo/ops/providers/npu/grouped_matmul.py:41-72``).

Pinned by: the textbook per-expert product on integer-valued inputs (exact in
fp32) and the fwd/bwd form of ``tests/ops/npu/test_grouped_matmul.py:11-90``
(counts ``[0, 5, 0, 11]``), see ``tests/test_oracle_kats.py``.
"""

from __future__ import annotations

import torch

from torchturbo_amd.dispatch import OpImpl, OpImplKind, register_op


def counts_list(tokens_per_expert) -> list[int]:
    if isinstance(tokens_per_expert, torch.Tensor):
        return [int(c) for c in tokens_per_expert.tolist()]
    return [int(c) for c in tokens_per_expert]


def grouped_matmul(x, weight, tokens_per_expert, *, trans_b: bool = False,
                   stacked_grad: bool = False):
    """``stacked_grad=False`` keeps the reference's autograd structure: one
    ``weight[e]`` per expert, whose backward allocates a full-size gradient
    buffer per expert (what the CPU baseline times). ``True`` takes the expert
    slices from one ``weight.unbind(0)``: the same gradient values with one
    full-size buffer, for checks of layers with many experts."""
    if weight.ndim != 3:
        raise ValueError(
            "grouped_matmul expects weight with shape (experts, in_features, out_features)."
        )
    counts = counts_list(tokens_per_expert)
    if len(counts) != weight.shape[0]:
        raise ValueError("tokens_per_expert must match the number of expert weight slices.")
    pieces = []
    begin = 0
    slices = weight.unbind(0) if stacked_grad else None
    for expert, n in enumerate(counts):
        if n:
            w = slices[expert] if stacked_grad else weight[expert]
            w = w.t() if trans_b else w
            pieces.append(x[begin:begin + n].matmul(w))
        begin += n
    if pieces:
        return torch.cat(pieces, dim=0)
    return x.new_empty((0, weight.shape[-2] if trans_b else weight.shape[-1]))


@register_op(op_name="grouped_matmul", impl_name="torch_grouped_matmul",
             kind=OpImplKind.NATIVE, priority=0, devices=())
class TorchGroupedMatmul(OpImpl):
    def __call__(self, x, weight, tokens_per_expert, *, trans_b: bool = False):
        return grouped_matmul(x, weight, tokens_per_expert, trans_b=trans_b)
