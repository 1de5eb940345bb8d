"""FP8 expert weights from an HF checkpoint, kept resident in e4m3.

The reference dequantises block-FP8 checkpoints (DeepSeek-V3 / Kimi / Ling:
e4m3 ``.weight`` with 128x128 ``.weight_scale_inv`` block scales, HF
``[out, in]`` orientation) to BF16 offline (``scripts/dequant/converter.py:35-127``,
``scripts/dequant/bailing.py:21-102``) and then assembles the expert tensors
(``src/torchturbo/models/weight_converter.py:417-449``). Here the e4m3 bytes and
the scales go straight into :class:`Fp8GroupedMLP` (``q1 [E, 2F, H]`` = gate rows
then up rows, ``q2 [E, H, F]`` = down, scales likewise), so the grouped GEMM
dequantises them on the fly; the expert keys are those of
``weight_converter.py:164-232``: ``{prefix}.{i}.{gate_proj|up_proj|down_proj}.weight``.

Checks follow ``bailing.py:57-102``: 2-D tensors, e4m3 weights, BF16 or FP32
scales of shape ``(ceil(out/128), ceil(in/128))``. Scales keep their dtype (the
kernels take either). BF16 master weights, when the module has them, receive
``bf16(f32(q) * f32(scale))`` — the reference's dequantised weight.
"""

from __future__ import annotations

import json
import math
from collections.abc import Mapping
from pathlib import Path

import torch

from .experts import Fp8GroupedMLP

BLOCK = 128
SCALE_SUFFIX = ".weight_scale_inv"


class SafetensorsCheckpoint(Mapping):
    """Lazy read-only view of a safetensors checkpoint: one file, or a directory
    with ``model.safetensors.index.json`` (sharded) or a single
    ``model.safetensors``. Tensors are read on access."""

    INDEX = "model.safetensors.index.json"

    def __init__(self, path: str | Path):
        from safetensors import safe_open  # lazy: only needed for loading

        self._open = safe_open
        path = Path(path).expanduser()
        if path.is_dir():
            index = path / self.INDEX
            if index.exists():
                with index.open(encoding="utf-8") as f:
                    weight_map = json.load(f)["weight_map"]
                self._files = {k: path / v for k, v in weight_map.items()}
            else:
                single = path / "model.safetensors"
                if not single.exists():
                    raise FileNotFoundError(f"no safetensors checkpoint in {path}")
                self._files = self._keys_of(single)
        elif path.exists():
            self._files = self._keys_of(path)
        else:
            raise FileNotFoundError(f"checkpoint not found: {path}")
        self._handles: dict[Path, object] = {}

    def _keys_of(self, file: Path) -> dict[str, Path]:
        with self._open(str(file), framework="pt") as f:
            return {k: file for k in f.keys()}

    def __getitem__(self, key: str) -> torch.Tensor:
        file = self._files[key]
        handle = self._handles.get(file)
        if handle is None:
            handle = self._handles[file] = self._open(str(file), framework="pt")
        return handle.get_tensor(key)

    def __iter__(self):
        return iter(self._files)

    def __len__(self) -> int:
        return len(self._files)


def _checked(name: str, weight: torch.Tensor, scale: torch.Tensor, shape: tuple[int, int]):
    if weight.dim() != 2:
        raise ValueError(f"{name}: weight must be a 2D tensor, got shape {tuple(weight.shape)}")
    if scale.dim() != 2:
        raise ValueError(f"{name}: scale must be a 2D tensor, got shape {tuple(scale.shape)}")
    if weight.dtype != torch.float8_e4m3fn:
        raise ValueError(f"{name}: unsupported weight dtype {weight.dtype}; expected FP8 E4M3")
    if scale.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"{name}: unsupported scale dtype {scale.dtype}; expected BF16 or FP32")
    if tuple(weight.shape) != shape:
        raise ValueError(f"{name}: weight shape {tuple(weight.shape)}, expected {shape}")
    want = (math.ceil(shape[0] / BLOCK), math.ceil(shape[1] / BLOCK))
    if tuple(scale.shape) != want:
        raise ValueError(f"{name}: scale shape {tuple(scale.shape)} does not match expected {want} "
                         f"for weight shape {shape} and block size {BLOCK}")
    return weight, scale


def dequantize_blocks(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """``bf16(f32(q) * f32(s))`` with ``s`` repeated over its 128x128 blocks; works on
    ``[..., R, C]`` weights with ``[..., ceil(R/128), ceil(C/128)]`` scales."""
    rows, cols = q.shape[-2:]
    s = scale.to(torch.float32).repeat_interleave(BLOCK, dim=-2).repeat_interleave(BLOCK, dim=-1)
    return (q.to(torch.float32) * s[..., :rows, :cols]).to(torch.bfloat16)


@torch.no_grad()
def load_fp8_experts(module: Fp8GroupedMLP, tensors: Mapping[str, torch.Tensor] | str | Path,
                     prefix: str, *, first_expert: int = 0, gate_name: str = "gate_proj",
                     up_name: str = "up_proj", down_name: str = "down_proj") -> None:
    """Fill ``module`` with experts ``first_expert .. first_expert + E - 1`` of the
    checkpoint (a mapping of tensors, or a safetensors file / directory path).

    ``prefix`` is the HF expert prefix, e.g. ``"model.layers.3.mlp.experts"``.
    """
    if not isinstance(tensors, Mapping):
        tensors = SafetensorsCheckpoint(tensors)
    E, two_f, H = module.q1.shape
    Fi = two_f // 2
    dev = module.q1.device

    def pair(i: int, proj: str, shape: tuple[int, int]):
        key = f"{prefix}.{i}.{proj}.weight"
        try:
            w, s = tensors[key], tensors[key[: -len(".weight")] + SCALE_SUFFIX]
        except KeyError as exc:
            raise KeyError(f"FP8 checkpoint has no tensor {exc.args[0]!r}") from None
        return _checked(key, w, s, shape)

    sdt = None
    for e in range(E):
        i = first_expert + e
        gq, gs = pair(i, gate_name, (Fi, H))
        uq, us = pair(i, up_name, (Fi, H))
        dq, ds = pair(i, down_name, (H, Fi))
        if sdt is None:
            sdt = gs.dtype
            for name in ("s1", "s2"):
                buf = getattr(module, name)
                if buf.dtype != sdt:  # keep the checkpoint's scale dtype (no rounding)
                    module.register_buffer(name, torch.empty(buf.shape, dtype=sdt, device=dev))
        if not (gs.dtype == us.dtype == ds.dtype == sdt):
            raise ValueError("FP8 checkpoint mixes scale dtypes across experts")
        module.q1[e, :Fi].copy_(gq)
        module.q1[e, Fi:].copy_(uq)
        module.s1[e, : Fi // BLOCK].copy_(gs)
        module.s1[e, Fi // BLOCK:].copy_(us)
        module.q2[e].copy_(dq)
        module.s2[e].copy_(ds)
    if module.master1 is not None:
        for e in range(E):  # one expert at a time (the fp32 expansion is 4 B per weight)
            module.master1[e].copy_(dequantize_blocks(module.q1[e], module.s1[e]))
            module.master2[e].copy_(dequantize_blocks(module.q2[e], module.s2[e]))
