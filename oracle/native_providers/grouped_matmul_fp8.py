"""Native FP8 block-scaled grouped matmul (CPU oracle).

The reference has no FP8 GEMM: its FP8 weights are dequantized offline to BF16
(``scripts/dequant/bailing.py:57-102``) and then used as ordinary BF16 expert
weights. This op restates exactly that composition: dequantize every expert
weight with the block-scale rule, then run the native grouped matmul with
``trans_b`` (weights stay in their HF ``[out, in]`` orientation, which is the
orientation the block scales are defined on).

``master`` (optional, [E, N, K]) receives the weight gradient: its forward
value is ignored and the gradient is the one of the dequantized BF16 weight.

Pinned by: the dequant KATs (``oracle/fp8.py``) and the grouped-matmul pins.
"""

from __future__ import annotations

import torch

from torchturbo_amd.dispatch import OpImpl, OpImplKind, register_op

from ..fp8 import dequantize_experts
from .grouped_matmul import grouped_matmul


class _DequantWithMasterGrad(torch.autograd.Function):
    @staticmethod
    def forward(ctx, master, deq):
        return deq

    @staticmethod
    def backward(ctx, grad):
        return grad, None


def grouped_matmul_fp8(x, qweight, scale, tokens_per_expert, *, master=None,
                       stacked_grad=False):
    deq = dequantize_experts(qweight, scale)
    if master is not None:
        deq = _DequantWithMasterGrad.apply(master, deq)
    return grouped_matmul(x, deq, tokens_per_expert, trans_b=True, stacked_grad=stacked_grad)


@register_op(op_name="grouped_matmul_fp8", impl_name="torch_grouped_matmul_fp8",
             kind=OpImplKind.NATIVE, priority=0, devices=())
class TorchGroupedMatmulFp8(OpImpl):
    def __call__(self, x, qweight, scale, tokens_per_expert, *, master=None):
        return grouped_matmul_fp8(x, qweight, scale, tokens_per_expert, master=master)
