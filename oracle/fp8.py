"""FP8 e4m3 weights with 128x128 block scales (CPU oracle).

``dequantize_weight`` restates the Ling/DeepSeek block format of
``scripts/dequant/bailing.py:57-102`` with ``Dequantizer.apply_scales_to_bf16``
(``scripts/dequant/dequantize.py:62-78``):
``W = bf16(fp32(q) * fp32(repeat_interleave(s, 128, both dims)[:R, :C]))``;
``weight_scale_inv`` is multiplied, not divided.

``quantize_blockwise`` is the synthetic-input generator for the FP8
configuration: per 128x128 block ``s = bf16(amax / 448)`` (``s = 1`` for an
all-zero block) and ``q = e4m3fn(W / s)``. It is not part of the reference;
it only has to be deterministic.

Pinned by: the KATs of ``tests/scripts/test_dequant.py:61-76`` (``[1, 2] x
[0.5, 2] = [0.5, 4]``), ``:144-153`` (``1 x 2``), ``:200-238`` (partial 33x33
and whole 128x128 blocks) restated in ``tests/test_oracle_kats.py``, and the
exhaustive decode of all 256 e4m3fn codes against the OCP E4M3 definition
(sign, 4-bit exponent with bias 7, 3-bit mantissa, subnormals, NaN at
S.1111.111, no infinities).
"""

from __future__ import annotations

import math

import torch

BLOCK = 128
E4M3_MAX = 448.0


def expand_block_scales(scale: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    want = (math.ceil(rows / BLOCK), math.ceil(cols / BLOCK))
    if tuple(scale.shape) != want:
        raise ValueError(
            f"Scale shape {tuple(scale.shape)} does not match expected {want} "
            f"for weight shape {(rows, cols)} and block size {BLOCK}"
        )
    full = scale.to(torch.float32).repeat_interleave(BLOCK, dim=1).repeat_interleave(BLOCK, dim=0)
    return full[:rows, :cols]


def dequantize_weight(weight: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    if weight.dim() != 2 or scale.dim() != 2:
        raise ValueError("expected 2-D weight and scale")
    if weight.dtype != torch.float8_e4m3fn:
        raise ValueError(f"Unsupported weight dtype {weight.dtype}; expected FP8 E4M3")
    if scale.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"Unsupported scale dtype {scale.dtype}; expected BF16 or FP32")
    s = expand_block_scales(scale, *weight.shape)
    return weight.to(torch.float32).mul(s).to(torch.bfloat16).contiguous()


def dequantize_experts(qweight: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """[E, R, C] e4m3fn + [E, R/128, C/128] scales -> [E, R, C] bf16."""
    return torch.stack([dequantize_weight(qweight[e], scale[e]) for e in range(qweight.shape[0])]) \
        if qweight.shape[0] else torch.empty(qweight.shape, dtype=torch.bfloat16)


def quantize_blockwise(weight: torch.Tensor, scale_dtype=torch.bfloat16):
    """[R, C] -> (e4m3fn [R, C], scales [ceil(R/128), ceil(C/128)])."""
    rows, cols = weight.shape
    br, bc = math.ceil(rows / BLOCK), math.ceil(cols / BLOCK)
    w = weight.to(torch.float32)
    pad = torch.zeros(br * BLOCK, bc * BLOCK)
    pad[:rows, :cols] = w
    blocks = pad.view(br, BLOCK, bc, BLOCK).abs().amax(dim=(1, 3))
    scale = torch.where(blocks > 0, blocks / E4M3_MAX, torch.ones_like(blocks)).to(scale_dtype)
    s = expand_block_scales(scale, rows, cols)
    q = (w / s).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return q, scale


def quantize_experts(weight: torch.Tensor, scale_dtype=torch.bfloat16):
    qs, ss = zip(*(quantize_blockwise(weight[e], scale_dtype) for e in range(weight.shape[0])))
    return torch.stack(qs), torch.stack(ss)


def e4m3fn_decode(code: int) -> float:
    """Value of one OCP E4M3 (fn) byte from its definition."""
    sign = -1.0 if code & 0x80 else 1.0
    exp = (code >> 3) & 0xF
    man = code & 0x7
    if exp == 0xF and man == 0x7:
        return math.nan
    if exp == 0:
        return sign * (man / 8.0) * 2.0 ** (1 - 7)
    return sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)
