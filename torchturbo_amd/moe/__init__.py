"""MoE layer stack (router, EP=1 token dispatcher, grouped experts)."""

from .experts import Fp8GroupedMLP, GroupedMLP
from .fp8_checkpoint import SafetensorsCheckpoint, load_fp8_experts
from .lora import GroupedLoRALinear, GroupedMLPLoRA
from .module import ModuleSpec, build_module
from .moe_config import MoEConfig, get_base_moe_config
from .moe_layer import MoELayer, MoERuntimeInputs, MoESubmodules
from .router import MoEAuxLossAutoScaler, RouterGatingLinearFunction, TopKRouter
from .token_dispatcher import MoEAlltoAllTokenDispatcher

__all__ = [
    "Fp8GroupedMLP",
    "GroupedLoRALinear",
    "GroupedMLP",
    "GroupedMLPLoRA",
    "MoEAlltoAllTokenDispatcher",
    "MoEAuxLossAutoScaler",
    "MoEConfig",
    "MoELayer",
    "MoERuntimeInputs",
    "MoESubmodules",
    "ModuleSpec",
    "RouterGatingLinearFunction",
    "SafetensorsCheckpoint",
    "TopKRouter",
    "build_module",
    "get_base_moe_config",
    "load_fp8_experts",
]
