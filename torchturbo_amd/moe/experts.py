"""Expert MLPs over expert-major packed rows.

``GroupedMLP`` mirrors ``src/torchturbo/models/modules/moe/experts.py:35-266``:

* ``weight1`` is ``[E*H, 2F]`` viewed ``[E, H, 2F]`` with the gate in columns
  ``[0, F)`` and up in ``[F, 2F)``; ``weight2`` is ``[E*F, H]`` viewed
  ``[E, F, H]`` (HF ``cat(gate, up).T`` / ``down.T``,
  ``src/torchturbo/models/weight_converter.py:417-449``);
* fc1 -> SwiGLU -> ``(act * probs).to(act.dtype)`` -> fc2, the probability
  product formed in the probs dtype (``experts.py:181-186``); on the GPU the
  SwiGLU and the weighting are one fused op (``swiglu_probs``), and so are the
  GELU / capped gates (``gated_activation_probs``, ``experts.py:52-84``);
* ``moe_apply_probs_on_input`` (top-1 only) scales the inputs instead;
* an empty input still produces (zero) weight gradients.

``Fp8GroupedMLP`` is the blockwise-FP8 variant: e4m3 expert weights with
128x128 block scales in HF ``[out, in]`` orientation (``q1 [E, 2F, H]``,
``q2 [E, H, F]``), dequantized inside the GEMM's operand staging. Optional
BF16 master weights of the same shape receive the weight gradients (the
gradient of the dequantized weight) and can be re-quantized after an
optimizer step with :meth:`Fp8GroupedMLP.requantize`.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch.nn.parameter import Parameter

from ..dispatch import ops
from .moe_config import MoEConfig


class GroupedMLP(torch.nn.Module):
    def __init__(self, num_local_experts: int, use_te: bool, config: MoEConfig,
                 layer_number: int | None = None):
        super().__init__()
        self.config = config
        self.num_local_experts = num_local_experts
        self.layer_number = layer_number
        limits = getattr(config, "moe_swiglu_limit", None)
        if limits is not None and layer_number is not None and 0 <= layer_number < len(limits):
            self.swiglu_limit = float(limits[layer_number])
        else:
            self.swiglu_limit = 0.0
        if self.swiglu_limit < 0:
            raise ValueError("moe_swiglu_limit must be non-negative.")
        if config.gated_linear_unit and config.activation_func not in (F.silu, F.gelu):
            raise ValueError("Activation function must be silu or gelu when using GroupedMLP.")
        self.use_te = use_te
        fc1_out = config.moe_ffn_hidden_size * (2 if config.gated_linear_unit else 1)
        self.weight1 = Parameter(torch.empty(config.hidden_size * num_local_experts, fc1_out,
                                             dtype=config.params_dtype))
        self.weight2 = Parameter(torch.empty(config.moe_ffn_hidden_size * num_local_experts,
                                             config.hidden_size, dtype=config.params_dtype))

    @property
    def _fused_swiglu(self) -> bool:
        return (self.config.gated_linear_unit and self.config.activation_func is F.silu
                and self.swiglu_limit == 0.0)

    def activation_func(self, x):
        if self.config.gated_linear_unit:
            if self._fused_swiglu:
                return ops.swiglu(x)
            return ops.gated_activation(
                x, activation_func=self.config.activation_func, limit=self.swiglu_limit,
                clamp_gate_after_activation=self.config.moe_swiglu_clamp_gate_after_activation,
            )
        return self.config.activation_func(x)

    def activation_func_with_probs(self, hidden_states, probs):
        """``(act(h) * probs).to(act.dtype)``; ``probs`` is [M] or [M, 1]."""
        flat = probs.reshape(-1)
        if self._fused_swiglu:
            return ops.swiglu_probs(hidden_states, flat)
        if self.config.gated_linear_unit:
            return ops.gated_activation_probs(
                hidden_states, flat, activation_func=self.config.activation_func,
                limit=self.swiglu_limit,
                clamp_gate_after_activation=self.config.moe_swiglu_clamp_gate_after_activation,
            )
        act = self.activation_func(hidden_states)
        return (act * flat.unsqueeze(-1)).to(act.dtype)

    def forward(self, permuted_local_hidden_states, tokens_per_expert, permuted_probs):
        x = permuted_local_hidden_states
        if self.config.moe_apply_probs_on_input:
            assert self.config.moe_router_topk == 1, \
                "`moe_apply_probs_on_input` only works with `moe_router_topk`=1."
            x = (permuted_probs.unsqueeze(-1) * x).to(x.dtype)
            permuted_probs = torch.ones_like(permuted_probs)
        if x.nelement() == 0:
            # No rows for these experts: dense products over the weight views keep
            # both weights in the graph, so they still receive (zero) gradients
            # (experts.py:255-264).
            h = torch.matmul(x, self.weight1.view(self.config.hidden_size, -1))
            h = self.activation_func_with_probs(h, permuted_probs)
            return torch.matmul(h, self.weight2.view(-1, self.config.hidden_size)), None
        w1 = self.weight1.view(self.num_local_experts, self.config.hidden_size, -1)
        w2 = self.weight2.view(self.num_local_experts, -1, self.config.hidden_size)
        fc1 = ops.grouped_matmul(x, w1, tokens_per_expert, trans_b=False)
        act = self.activation_func_with_probs(fc1, permuted_probs)
        fc2 = ops.grouped_matmul(act, w2, tokens_per_expert, trans_b=False)
        return fc2, None


class Fp8GroupedMLP(torch.nn.Module):
    """SwiGLU experts with e4m3 weights and 128x128 block scales."""

    def __init__(self, num_local_experts: int, use_te: bool, config: MoEConfig,
                 layer_number: int | None = None, with_master: bool = True):
        super().__init__()
        if not (config.gated_linear_unit and config.activation_func is F.silu):
            raise ValueError("Fp8GroupedMLP implements SwiGLU experts only.")
        self.config = config
        self.num_local_experts = num_local_experts
        E, H, Fi = num_local_experts, config.hidden_size, config.moe_ffn_hidden_size
        if H % 128 or Fi % 128:
            raise ValueError("FP8 block scales need hidden and ffn sizes divisible by 128.")
        self.register_buffer("q1", torch.zeros(E, 2 * Fi, H, dtype=torch.float8_e4m3fn))
        self.register_buffer("s1", torch.ones(E, 2 * Fi // 128, H // 128, dtype=torch.bfloat16))
        self.register_buffer("q2", torch.zeros(E, H, Fi, dtype=torch.float8_e4m3fn))
        self.register_buffer("s2", torch.ones(E, H // 128, Fi // 128, dtype=torch.bfloat16))
        if with_master:
            self.master1 = Parameter(torch.zeros(E, 2 * Fi, H, dtype=torch.bfloat16))
            self.master2 = Parameter(torch.zeros(E, H, Fi, dtype=torch.bfloat16))
        else:
            self.master1 = None
            self.master2 = None

    def load_quantized(self, q1, s1, q2, s2):
        with torch.no_grad():
            self.q1.copy_(q1)
            self.s1.copy_(s1)
            self.q2.copy_(q2)
            self.s2.copy_(s2)

    def requantize(self):
        """Quantize the master weights into ``q``/``s`` (128x128 blocks, s = amax/448)."""
        if self.master1 is None:
            raise RuntimeError("no master weights to quantize")
        with torch.no_grad():
            for master, q, s in ((self.master1, self.q1, self.s1), (self.master2, self.q2, self.s2)):
                E, R, C = master.shape
                blocks = master.float().view(E, R // 128, 128, C // 128, 128).abs().amax(dim=(2, 4))
                scale = torch.where(blocks > 0, blocks / 448.0, torch.ones_like(blocks)).to(s.dtype)
                full = scale.float().repeat_interleave(128, 1).repeat_interleave(128, 2)
                q.copy_((master.float() / full).clamp(-448.0, 448.0).to(torch.float8_e4m3fn))
                s.copy_(scale)

    def forward(self, permuted_local_hidden_states, tokens_per_expert, permuted_probs):
        fc1 = ops.grouped_matmul_fp8(permuted_local_hidden_states, self.q1, self.s1,
                                     tokens_per_expert, master=self.master1)
        act = ops.swiglu_probs(fc1, permuted_probs.reshape(-1))
        fc2 = ops.grouped_matmul_fp8(act, self.q2, self.s2, tokens_per_expert,
                                     master=self.master2)
        return fc2, None
