"""HIP grouped GEMM providers (bf16/f16 MFMA, f32; FP8 block-scaled weights).

``grouped_matmul`` keeps the reference contract
(``src/torchturbo/ops/providers/native/grouped_matmul.py:16-56``): weight
``[E, K, N]`` (``[E, N, K]`` with ``trans_b``), per-expert row counts as a
list, a CPU tensor or a device tensor; empty experts contribute no rows and
get zero weight gradients. Counts on the device are used in place (no host
synchronisation).

``grouped_matmul_fp8`` takes e4m3 weights ``qweight [E, N, K]`` in HF
``[out, in]`` orientation with 128x128 block scales ``[E, N/128, K/128]``
(bf16 or f32); the weight gradient (of the dequantized bf16 weight) flows to
``master`` when given.
"""

from __future__ import annotations

import torch

from ...dispatch import OpImpl, OpImplKind, register_op
from ...runtime import TurboDevice
from . import PRIORITY
from ._functions import GroupedMatmul, GroupedMatmulFp8, device_counts, require_cuda
from .available import hip_available


@register_op(op_name="grouped_matmul", impl_name="hip_grouped_matmul",
             kind=OpImplKind.CUSTOM, priority=PRIORITY, devices=(TurboDevice.CUDA,))
class HipGroupedMatmul(OpImpl):
    def available(self) -> bool:
        return hip_available()

    def __call__(self, x, weight, tokens_per_expert, *, trans_b: bool = False):
        if weight.ndim != 3:
            raise ValueError(
                "grouped_matmul expects weight with shape (experts, in_features, out_features)."
            )
        dev = require_cuda(x, weight)
        counts = device_counts(tokens_per_expert, weight.shape[0], dev, m=x.shape[0])
        return GroupedMatmul.apply(x, weight, counts, bool(trans_b))


@register_op(op_name="grouped_matmul_fp8", impl_name="hip_grouped_matmul_fp8",
             kind=OpImplKind.CUSTOM, priority=PRIORITY, devices=(TurboDevice.CUDA,))
class HipGroupedMatmulFp8(OpImpl):
    def available(self) -> bool:
        return hip_available()

    def __call__(self, x, qweight, scale, tokens_per_expert, *, master=None):
        if qweight.ndim != 3 or qweight.dtype != torch.float8_e4m3fn:
            raise ValueError("grouped_matmul_fp8 expects float8_e4m3fn weights [E, N, K].")
        E, N, K = qweight.shape
        want = (E, -(-N // 128), -(-K // 128))
        if tuple(scale.shape) != want:
            raise ValueError(f"scale shape {tuple(scale.shape)} does not match {want}")
        if master is not None and tuple(master.shape) != (E, N, K):
            raise ValueError("master weight must have the shape of qweight")
        dev = require_cuda(x, qweight, scale, master)
        counts = device_counts(tokens_per_expert, E, dev, m=x.shape[0])
        return GroupedMatmulFp8.apply(x, master, qweight.view(torch.uint8), scale, counts)
