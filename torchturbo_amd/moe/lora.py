"""Per-expert LoRA adapters on the grouped expert MLP.

Mirrors ``src/torchturbo/engine/peft/lora.py:54-725``:

* ``GroupedLoRALinear`` (``lora.py:54-125``) holds one fp32 matrix per expert,
  ``[E, in, out]``, and multiplies expert-major packed rows by it with the
  ``grouped_matmul`` op (the same grouped GEMM as the base layer);
* ``GroupedMLPLoRA`` (``lora.py:128-725``) wraps a :class:`GroupedMLP` and adds
  ``scaling * gmm(gmm(dropout(x).float(), A), B).to(out.dtype)`` to its fc1 and
  fc2 outputs (additive residual, no ``[E, in, out]`` delta is formed), with
  the reference's adapter management: ranks, ``lora_alpha`` scaling (plain or
  rank-stabilised), dropout, Kaiming-uniform or Gaussian initialisation, active
  adapter selection, merge / unmerge into the base weights and the conversion
  of legacy 2-D LoRA checkpoints (``lora.py:245-319``).

The reference builds on PEFT's ``BaseTunerLayer``; here the class derives from
it when PEFT is importable and works standalone otherwise (PEFT's adapter
bookkeeping then reduces to the methods defined below).
"""

from __future__ import annotations

import math
from typing import Any, Optional, Union

import torch
import torch.nn as nn

from ..dispatch import ops
from .experts import GroupedMLP

try:  # PEFT integration is optional (the reference requires it)
    from peft.tuners.tuners_utils import BaseTunerLayer as _TunerBase
    from peft.tuners.tuners_utils import check_adapters_to_merge as _peft_check
except ImportError:  # pragma: no cover - depends on the environment
    _TunerBase = object
    _peft_check = None


def _adapters_to_merge(layer, adapter_names):
    if _peft_check is not None:
        return _peft_check(layer, adapter_names)
    names = layer.active_adapters if adapter_names is None else list(adapter_names)
    return [n for n in names if n not in layer.merged_adapters]


class GroupedLoRALinear(nn.Module):
    """One fp32 ``[in, out]`` matrix per local expert, applied by grouped GEMM."""

    def __init__(self, num_experts: int, in_features: int, out_features: int,
                 dtype: torch.dtype = torch.float32) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.empty(num_experts, in_features, out_features, dtype=dtype))
        self.num_experts = num_experts
        self.in_features = in_features
        self.out_features = out_features

    def forward(self, x: torch.Tensor, tokens_per_expert: torch.Tensor) -> torch.Tensor:
        return ops.grouped_matmul(x, self.weight, tokens_per_expert, trans_b=False)

    def __repr__(self) -> str:
        return (f"{self.__class__.__name__}(num_experts={self.num_experts}, "
                f"in_features={self.in_features}, out_features={self.out_features})")


class GroupedMLPLoRA(nn.Module, _TunerBase):
    """LoRA wrapper of :class:`GroupedMLP` with additive-residual grouped GEMMs."""

    adapter_layer_names = ("lora_A", "lora_B", "lora_A2", "lora_B2")
    other_param_names = ("r", "lora_alpha", "scaling", "lora_dropout")

    def __init__(self, base_layer: GroupedMLP, adapter_name: str, r: int = 0,
                 lora_alpha: int = 1, lora_dropout: float = 0.0,
                 init_lora_weights: Union[bool, str] = True, use_rslora: bool = False,
                 use_dora: bool = False, lora_bias: bool = False, **kwargs) -> None:
        nn.Module.__init__(self)
        if use_dora:
            raise ValueError("GroupedMLPLoRA does not support DoRA (use_dora=True).")
        if lora_bias:
            raise ValueError("GroupedMLPLoRA does not support lora_bias=True.")
        self.base_layer = base_layer
        self.num_local_experts = base_layer.num_local_experts
        self.config = cfg = base_layer.config
        ffn = cfg.moe_ffn_hidden_size
        # Per-expert [in, out] shapes of weight1 (gate | up) and weight2 (down).
        self.in_features_weight1 = cfg.hidden_size
        self.out_features_weight1 = ffn * (2 if cfg.gated_linear_unit else 1)
        self.in_features_weight2 = ffn
        self.out_features_weight2 = cfg.hidden_size
        self.in_features = cfg.hidden_size
        self.out_features = cfg.hidden_size

        self.r: dict[str, int] = {}
        self.lora_alpha: dict[str, int] = {}
        self.scaling: dict[str, float] = {}
        self.lora_dropout = nn.ModuleDict({})
        self.lora_A = nn.ModuleDict({})
        self.lora_B = nn.ModuleDict({})
        self.lora_A2 = nn.ModuleDict({})
        self.lora_B2 = nn.ModuleDict({})
        self._disable_adapters = False
        self.merged_adapters: list[str] = []
        self.use_dora: dict[str, bool] = {}
        self.lora_bias: dict[str, bool] = {}
        self.lora_magnitude_vector = nn.ModuleDict()
        self._caches: dict[str, Any] = {}
        self.ephemeral_gpu_offload = False
        self.cast_input_dtype_enabled = True
        self.kwargs = kwargs
        self._active_adapter = adapter_name
        self.update_layer(adapter_name, r, lora_alpha=lora_alpha, lora_dropout=lora_dropout,
                          init_lora_weights=init_lora_weights, use_rslora=use_rslora,
                          use_dora=use_dora, lora_bias=lora_bias)

    # -- legacy checkpoints ---------------------------------------------------
    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        self._convert_legacy_weights(state_dict, prefix)
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)

    def _convert_legacy_weights(self, state_dict: dict, prefix: str) -> None:
        """2-D ``nn.Linear`` LoRA weights -> the 3-D per-expert layout.

        A: ``[r*E, in]`` (expert-major rows) -> ``[E, in, r]``;
        B: ``[out, r*E]`` -> ``[E, r, out]`` with ``new[e, k, o] = old[o, e*r + k]``,
        the layouts stated at ``lora.py:273-286``. (The reference's own B branch,
        ``old.T.view(E, out, r)``, raises on the transposed view.)
        """
        n = self.num_local_experts
        for name, r in self.r.items():
            for key, is_b, fin, fout in (
                (f"lora_A.{name}.weight", False, self.in_features_weight1, r),
                (f"lora_B.{name}.weight", True, r, self.out_features_weight1),
                (f"lora_A2.{name}.weight", False, self.in_features_weight2, r),
                (f"lora_B2.{name}.weight", True, r, self.out_features_weight2),
            ):
                full = prefix + key
                old = state_dict.get(full)
                if old is None or old.dim() != 2:
                    continue
                if is_b:
                    state_dict[full] = old.T.reshape(n, fin, fout).contiguous()
                else:
                    state_dict[full] = old.reshape(n, fout, fin).permute(0, 2, 1).contiguous()

    # -- adapter bookkeeping --------------------------------------------------
    @property
    def active_adapter(self) -> str:
        return self._active_adapter

    @active_adapter.setter
    def active_adapter(self, value: str) -> None:
        self._active_adapter = value

    @property
    def active_adapters(self) -> list[str]:
        a = self._active_adapter
        return [a] if isinstance(a, str) else list(a)

    @property
    def disable_adapters(self) -> bool:
        return self._disable_adapters

    @property
    def merged(self) -> bool:
        return bool(self.merged_adapters)

    def set_adapter(self, adapter_names: Union[str, list[str]]) -> None:
        names = [adapter_names] if isinstance(adapter_names, str) else list(adapter_names)
        for name in names:
            if name not in self.r:
                raise ValueError(f"Adapter {name!r} not found in GroupedMLPLoRA. "
                                 f"Available: {list(self.r.keys())}")
        self._active_adapter = names[0] if len(names) == 1 else names

    def enable_adapters(self, enabled: bool) -> None:
        self._disable_adapters = not enabled

    def get_base_layer(self) -> nn.Module:
        return self.base_layer

    def update_layer(self, adapter_name: str, r: int, lora_alpha: int, lora_dropout: float,
                     init_lora_weights: Union[bool, str], use_rslora: bool = False,
                     use_dora: bool = False, use_qalora: bool = False, lora_bias: bool = False,
                     qalora_group_size: int = 32, **kwargs) -> None:
        if r <= 0:
            raise ValueError(f"`r` should be a positive integer, got {r}")
        if use_dora:
            raise ValueError("GroupedMLPLoRA does not support DoRA.")
        if lora_bias:
            raise ValueError("GroupedMLPLoRA does not support lora_bias=True.")
        self.r[adapter_name] = r
        self.lora_alpha[adapter_name] = lora_alpha
        self.lora_dropout[adapter_name] = nn.Dropout(p=lora_dropout) if lora_dropout > 0.0 \
            else nn.Identity()
        n = self.num_local_experts
        # fp32 adapters whatever the base dtype (lora.py:426-440).
        self.lora_A[adapter_name] = GroupedLoRALinear(n, self.in_features_weight1, r)
        self.lora_B[adapter_name] = GroupedLoRALinear(n, r, self.out_features_weight1)
        self.lora_A2[adapter_name] = GroupedLoRALinear(n, self.in_features_weight2, r)
        self.lora_B2[adapter_name] = GroupedLoRALinear(n, r, self.out_features_weight2)
        self.lora_bias[adapter_name] = lora_bias
        self.scaling[adapter_name] = lora_alpha / (math.sqrt(r) if use_rslora else r)
        self.use_dora[adapter_name] = False
        a_w = (self.lora_A[adapter_name].weight, self.lora_A2[adapter_name].weight)
        b_w = (self.lora_B[adapter_name].weight, self.lora_B2[adapter_name].weight)
        if isinstance(init_lora_weights, str) and init_lora_weights.lower() == "gaussian":
            for w in a_w:
                nn.init.normal_(w, std=1 / r)
        elif init_lora_weights:
            for w in a_w:
                nn.init.kaiming_uniform_(w, a=math.sqrt(5))
        if init_lora_weights:
            for w in b_w:
                nn.init.zeros_(w)
        device = next(self.base_layer.parameters()).device
        for group in (self.lora_A, self.lora_B, self.lora_A2, self.lora_B2):
            group[adapter_name] = group[adapter_name].to(device)
        self.set_adapter(self.active_adapters)

    # -- merge / unmerge ------------------------------------------------------
    def _compute_deltas(self, adapter_names: Optional[list[str]] = None):
        """Sum over adapters of ``scaling * A @ B`` per expert: ([E, H, fc1], [E, ffn, H])."""
        d1 = d2 = None
        for name in (self.active_adapters if adapter_names is None else adapter_names):
            if name not in self.r:
                continue
            s = self.scaling[name]
            a1 = s * torch.matmul(self.lora_A[name].weight, self.lora_B[name].weight)
            a2 = s * torch.matmul(self.lora_A2[name].weight, self.lora_B2[name].weight)
            d1 = a1 if d1 is None else d1 + a1
            d2 = a2 if d2 is None else d2 + a2
        return d1, d2

    def merge(self, safe_merge: bool = False, adapter_names: Optional[list[str]] = None) -> None:
        for name in _adapters_to_merge(self, adapter_names):
            if name not in self.r:
                continue
            d1, d2 = self._compute_deltas([name])
            base = self.get_base_layer()
            if safe_merge:
                n1 = base.weight1.data.clone() + d1.view_as(base.weight1)
                n2 = base.weight2.data.clone() + d2.view_as(base.weight2)
                if not (torch.isfinite(n1).all() and torch.isfinite(n2).all()):
                    raise ValueError(f"NaNs detected in merged weights for adapter {name!r}")
                base.weight1.data = n1
                base.weight2.data = n2
            else:
                base.weight1.data += d1.view_as(base.weight1)
                base.weight2.data += d2.view_as(base.weight2)
            self.merged_adapters.append(name)

    def unmerge(self) -> None:
        while self.merged_adapters:
            name = self.merged_adapters.pop()
            if name not in self.r:
                continue
            d1, d2 = self._compute_deltas([name])
            base = self.get_base_layer()
            base.weight1.data -= d1.view_as(base.weight1)
            base.weight2.data -= d2.view_as(base.weight2)

    # -- forward --------------------------------------------------------------
    def _residual(self, x, counts, names, a_group, b_group, out_dtype):
        total = None
        for name in names:
            a, b = a_group[name], b_group[name]
            xd = self.lora_dropout[name](x).to(a.weight.dtype)
            delta = ops.grouped_matmul(ops.grouped_matmul(xd, a.weight, counts, trans_b=False),
                                       b.weight, counts, trans_b=False)
            term = delta.to(out_dtype) * self.scaling[name]
            total = term if total is None else total + term
        return total

    def forward(self, permuted_local_hidden_states: torch.Tensor,
                tokens_per_expert: torch.Tensor, permuted_probs: torch.Tensor, **kwargs):
        x, counts, probs = permuted_local_hidden_states, tokens_per_expert, permuted_probs
        if self._disable_adapters:
            if self.merged_adapters:
                self.unmerge()
            return self.base_layer(x, counts, probs)
        if self.merged_adapters:
            return self.base_layer(x, counts, probs)
        active = [a for a in self.active_adapters if a in self.r]
        if not active:
            return self.base_layer(x, counts, probs)
        base = self.base_layer
        E, H = base.num_local_experts, base.config.hidden_size
        if base.config.moe_apply_probs_on_input:
            assert base.config.moe_router_topk == 1, \
                "`moe_apply_probs_on_input` only works with `moe_router_topk`=1."
            x = (probs.unsqueeze(-1) * x).to(x.dtype)
            probs = torch.ones_like(probs)
        if x.nelement() == 0:
            # Keep every adapter in the graph so that all ranks produce (zero)
            # gradients for them (lora.py:705-719).
            zero = x.sum() * 0 + probs.sum() * 0
            for name in active:
                for group in (self.lora_A, self.lora_B, self.lora_A2, self.lora_B2):
                    zero = zero + group[name].weight.sum() * 0
            return torch.zeros_like(x) + zero, None
        w1 = base.weight1.view(E, H, -1)
        w2 = base.weight2.view(E, -1, H)
        fc1 = ops.grouped_matmul(x, w1, counts, trans_b=False)
        # Each adapter's residual is added in turn, as the reference does.
        for name in active:
            fc1 = fc1 + self._residual(x, counts, [name], self.lora_A, self.lora_B, fc1.dtype)
        act = base.activation_func_with_probs(fc1, probs.unsqueeze(-1))
        fc2 = ops.grouped_matmul(act, w2, counts, trans_b=False)
        for name in active:
            fc2 = fc2 + self._residual(act, counts, [name], self.lora_A2, self.lora_B2, fc2.dtype)
        return fc2, None

    def __repr__(self) -> str:
        return f"lora.GroupedMLPLoRA({super().__repr__()})"
