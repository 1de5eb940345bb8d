"""MoE layer configuration.

Same fields, defaults and validation as the reference's ``MoEConfig``
(``src/torchturbo/models/modules/moe/moe_config.py:22-87``).
"""

from __future__ import annotations

import functools
from dataclasses import dataclass
from typing import Callable, List, Optional

import torch
import torch.nn.functional as F


def init_method_normal(sigma):
    return functools.partial(torch.nn.init.normal_, mean=0.0, std=sigma)


@dataclass
class MoEConfig:
    hidden_size: int = 0
    gated_linear_unit: bool = False
    activation_func: Callable = F.gelu
    num_moe_experts: Optional[int] = None
    expert_model_parallel_size: int = 1
    params_dtype: torch.dtype = torch.float32
    perform_initialization: bool = True
    init_method: Optional[Callable] = None
    init_method_std: float = 0.02
    moe_shared_expert_intermediate_size: Optional[int] = None
    moe_ffn_hidden_size: Optional[int] = None
    moe_router_load_balancing_type: str = "none"
    moe_aux_loss_coeff: float = 0.0
    moe_z_loss_coeff: float = 0.0
    moe_router_topk: int = 2
    moe_router_num_groups: Optional[int] = None
    moe_router_group_topk: Optional[int] = None
    moe_router_pre_softmax: bool = False
    moe_router_topk_scaling_factor: Optional[float] = None
    moe_router_score_function: str = "softmax"
    moe_router_dtype: Optional[str] = None
    moe_router_enable_expert_bias: bool = False
    moe_token_dispatcher_type: str = "alltoall"
    moe_apply_probs_on_input: bool = False
    moe_swiglu_limit: Optional[List[float]] = None
    moe_swiglu_clamp_gate_after_activation: bool = False
    num_hash_layers: int = 0
    vocab_size: int = 0

    def __post_init__(self):
        if self.init_method is None:
            self.init_method = init_method_normal(self.init_method_std)
        if (self.moe_router_enable_expert_bias
                and self.moe_router_score_function == "softmax"
                and not self.moe_router_pre_softmax):
            raise ValueError(
                "Softmax expert bias requires moe_router_pre_softmax=True; "
                "post-top-k softmax would ignore the bias."
            )


def get_base_moe_config(hf_config, ep_size: int, **overrides) -> dict:
    """HF config -> ``MoEConfig`` kwargs (``config_converter.py:5-22``)."""
    kwargs = dict(
        hidden_size=hf_config.hidden_size,
        gated_linear_unit=True,
        activation_func=F.silu,
        expert_model_parallel_size=ep_size,
        moe_ffn_hidden_size=hf_config.moe_intermediate_size,
        moe_router_load_balancing_type="none",
        moe_router_topk=hf_config.num_experts_per_tok,
        moe_token_dispatcher_type="alltoall",
    )
    kwargs.update(overrides)
    return kwargs
