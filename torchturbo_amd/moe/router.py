"""Top-k router.

Mirrors ``TopKRouter`` (``src/torchturbo/models/modules/moe/router.py:25-380``):
the gating linear runs in the router dtype with autocast off and recomputes
its casts in backward (``:25-58``); ``routing`` applies the z-loss, calls the
top-k selection, attaches the aux loss and accumulates expert-bias counts
(``:277-356``). Top-k selection goes through the ``topk_softmax_with_capacity``
op, and the [T, E] sums behind the aux loss and the z-loss (per-expert score
sums and top-k counts of the bias-free scores, the sum of squared
log-sum-exps) through the ``router_loss_stats`` op, so the GPU runs one HIP
kernel for each per direction. The scalar formulas on top of those sums, the
sequence-parallel all-reduce and the metrics are the reference's
(``router.py:164-270``). ``compute_routing_scores_for_aux_loss`` and
``z_loss_func`` (``moe_utils.py:15-70``) remain importable.

``forward`` runs the gating linear and the top-k as one op
(``router_gate_topk``: one HIP kernel on the GPU) when the inputs and the
router weight share a 16-bit dtype, the router dtype is that dtype or fp32,
E is a multiple of 32 up to 256 and the hidden size a multiple of 64; the
z-loss is then attached to the probabilities instead of the logits the
top-k read (the same gradients: the loss scaler is an identity). Other
configurations run ``gating`` and ``routing`` as the reference does.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.distributed as dist

from ..dispatch import ops
from .moe_config import MoEConfig

# Sizes the HIP router kernels cover (tt_router_topk_fwd / _bwd,
# tt_router_loss_fwd: E <= 1024, k <= 64).
MAX_EXPERTS = 1024
MAX_TOPK = 64


def _op_resolves(name: str) -> bool:
    """Whether the process dispatcher has an implementation of ``name`` for its device."""
    from ..dispatch.ops import get_ops

    try:
        d = get_ops()
    except RuntimeError:
        return False
    return bool(d.registry.list(lambda s: s.op_name == name)) and name not in d.unresolved_ops


def _group_size(group) -> int:
    if group is None or not dist.is_available() or not dist.is_initialized():
        return 1
    return dist.get_world_size(group)


class MoEAuxLossAutoScaler(torch.autograd.Function):
    """Attach an auxiliary loss to an activation (``moe_utils.py:73-90``)."""

    loss_scale = 1.0

    @staticmethod
    def forward(ctx, output, aux_loss):
        ctx.save_for_backward(aux_loss)
        return output

    @staticmethod
    def backward(ctx, grad_output):
        (aux_loss,) = ctx.saved_tensors
        return grad_output, torch.ones_like(aux_loss) * MoEAuxLossAutoScaler.loss_scale

    @classmethod
    def set_loss_scale(cls, scale: float) -> None:
        cls.loss_scale = scale


def mask_padding_tokens(values, padding_mask):
    if padding_mask is None:
        return values
    return values * (~padding_mask.reshape(-1).bool()).unsqueeze(-1)


def compute_routing_scores_for_aux_loss(logits, topk, score_function, padding_mask=None):
    """Bias-free routing map and scores for the aux loss (``moe_utils.py:15-45``)."""
    logits = logits.reshape(-1, logits.size(-1))
    if score_function == "softmax":
        scores = torch.softmax(logits, dim=-1, dtype=torch.float32)
    elif score_function in ("sigmoid", "sqrtsoftplus"):
        scores = (torch.sigmoid(logits.float()) if score_function == "sigmoid"
                  else torch.nn.functional.softplus(logits.float()).sqrt())
        scores = scores / (scores.sum(dim=-1, keepdim=True) + 1e-20)
    else:
        raise ValueError(f"Invalid score_function: {score_function}")
    top = torch.topk(scores, k=topk, dim=-1).indices
    routing_map = torch.zeros_like(logits, dtype=torch.int32).scatter_(1, top, 1).bool()
    if padding_mask is not None:
        scores = mask_padding_tokens(scores, padding_mask)
        routing_map = mask_padding_tokens(routing_map, padding_mask).bool()
    return routing_map, scores


def z_loss_func(logits, z_loss_coeff, padding_mask=None):
    """Mean squared logsumexp over valid tokens (``moe_utils.py:48-70``)."""
    values = torch.square(torch.logsumexp(logits, dim=-1))
    if padding_mask is not None:
        valid = ~padding_mask.reshape(-1).bool()
        z = (values * valid).sum() / torch.clamp(valid.sum(), min=1)
    else:
        z = values.sum() if logits.shape[0] == 0 else values.mean()
    return z * z_loss_coeff


class RouterGatingLinearFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, input, weight, router_dtype):
        ctx.save_for_backward(input, weight)
        ctx.router_dtype = router_dtype
        with torch.autocast(device_type=input.device.type, enabled=False):
            return torch.nn.functional.linear(input.to(router_dtype), weight.to(router_dtype))

    @staticmethod
    def backward(ctx, grad_output):
        input, weight = ctx.saved_tensors
        grad_output = grad_output.reshape(-1, grad_output.shape[-1])
        grad_input = grad_weight = None
        if ctx.needs_input_grad[0]:
            grad_input = grad_output.mm(weight.to(ctx.router_dtype))
            grad_input = grad_input.view(input.shape).to(input.dtype)
        if ctx.needs_input_grad[1]:
            flat = input.reshape(-1, input.shape[-1]).to(ctx.router_dtype)
            grad_weight = grad_output.t().mm(flat).to(weight.dtype)
        return grad_input, grad_weight, None


class Router(torch.nn.Module):
    def __init__(self, config: MoEConfig) -> None:
        super().__init__()
        self.config = config
        self.num_experts = config.num_moe_experts
        self.layer_number = None
        self.weight = torch.nn.Parameter(
            torch.empty((config.num_moe_experts, config.hidden_size), dtype=torch.float32)
        )
        if config.perform_initialization:
            config.init_method(self.weight)
        self.weight.data = self.weight.data.to(dtype=config.params_dtype)

    def router_dtype(self, input_dtype):
        if self.config.moe_router_dtype == "fp32":
            return torch.float32
        if self.config.moe_router_dtype == "fp64":
            return torch.float64
        return input_dtype

    def gating(self, input):
        if self.weight.device != input.device:
            self.weight.data = self.weight.data.to(device=input.device)
        return RouterGatingLinearFunction.apply(input, self.weight, self.router_dtype(input.dtype))


class TopKRouter(Router):
    def __init__(self, config: MoEConfig, layer_number: Optional[int] = None, sp_group=None):
        super().__init__(config=config)
        # Limits of the HIP top-k kernels (one wave per token, up to 16 experts
        # per lane, a k-round selection), stated here so that a layer the GPU
        # cannot route fails when it is built, not on its first call. Router
        # dtypes fp32, fp64 and the input dtype are all supported.
        if config.num_moe_experts > MAX_EXPERTS:
            raise ValueError(f"TopKRouter: num_moe_experts={config.num_moe_experts} exceeds the "
                             f"{MAX_EXPERTS} experts the router kernels support")
        if config.moe_router_topk > MAX_TOPK:
            raise ValueError(f"TopKRouter: moe_router_topk={config.moe_router_topk} exceeds the "
                             f"{MAX_TOPK} the router kernels support")
        self.topk = config.moe_router_topk
        self.routing_type = config.moe_router_load_balancing_type
        self.score_function = config.moe_router_score_function
        self.layer_number = layer_number
        self.sp_group = sp_group
        self._metrics = None
        self.use_hash_routing = (layer_number is not None and layer_number < config.num_hash_layers
                                 and config.vocab_size > 0)
        self.enable_expert_bias = config.moe_router_enable_expert_bias and not self.use_hash_routing
        if self.enable_expert_bias:
            self.register_buffer("expert_bias",
                                 torch.zeros(config.num_moe_experts, dtype=torch.float32))
        else:
            self.expert_bias = None
        if self.use_hash_routing:
            self.register_buffer("tid2eid", torch.stack([
                torch.randperm(config.num_moe_experts)[: self.topk]
                for _ in range(config.vocab_size)
            ]).long())

    def _maintain_float32_expert_bias(self):
        if getattr(self, "expert_bias", None) is not None and self.expert_bias.dtype != torch.float32:
            self.expert_bias.data = self.expert_bias.data.to(torch.float32)

    def _apply_aux_loss(self, probs, prob_sum, tokens_per_expert):
        """``router.py:180-223`` with ``prob_sum = scores.sum(0)`` and
        ``tokens_per_expert = routing_map.sum(0)`` already reduced
        (``router_loss_stats``)."""
        coeff = self.config.moe_aux_loss_coeff
        if coeff == 0.0:
            return probs
        sp_size = _group_size(self.sp_group)
        if sp_size > 1:
            dist.all_reduce(tokens_per_expert, op=dist.ReduceOp.SUM, group=self.sp_group)
        total = (tokens_per_expert.sum() / self.topk).clamp_min(1)
        raw = (torch.sum(prob_sum * tokens_per_expert) * self.num_experts * sp_size
               / (self.topk * total * total))
        aux = raw * coeff
        self._metrics = {**(self._metrics or {}), "aux_loss": (aux / coeff).detach(),
                         "aux_loss_scaled": aux.detach()}
        return MoEAuxLossAutoScaler.apply(probs, aux)

    def apply_z_loss(self, logits, padding_mask=None, z_sum=None):
        """``router.py:225-270``; the local z-loss is ``z_loss_func``'s mean of
        the squared log-sum-exps, formed from their sum ``z_sum`` (computed here
        through ``router_loss_stats`` when not given)."""
        if not self.config.moe_z_loss_coeff or not (self.training and torch.is_grad_enabled()):
            return logits
        return MoEAuxLossAutoScaler.apply(logits, self._z_loss(logits, padding_mask, z_sum))

    def _z_loss(self, logits, padding_mask, z_sum=None):
        """The scaled z-loss of ``router.py:239-264`` (metrics recorded)."""
        coeff = self.config.moe_z_loss_coeff
        if z_sum is None:
            z_sum = ops.router_loss_stats(logits, self.topk, self.score_function, padding_mask,
                                          aux=False, z=True)[2]
        if padding_mask is not None:
            local = (~padding_mask.reshape(-1).bool()).sum()
            local_z = z_sum.to(logits.dtype) / torch.clamp(local, min=1)
        else:
            local = torch.tensor(logits.shape[0], device=logits.device, dtype=torch.long)
            local_z = (z_sum / max(logits.shape[0], 1)).to(logits.dtype)
        total = local.clone()
        sp_size = _group_size(self.sp_group)
        if sp_size > 1:
            dist.all_reduce(total, op=dist.ReduceOp.SUM, group=self.sp_group)
        z = local_z * coeff * (sp_size * local / torch.clamp(total, min=1))
        self._metrics = {**(self._metrics or {}), "z_loss": (z / coeff).detach(),
                         "z_loss_scaled": z.detach()}
        return z

    def pop_metrics(self):
        metrics = self._metrics or {}
        self._metrics = None
        return metrics

    def _routing_kwargs(self, input_ids):
        return dict(
            use_pre_softmax=self.config.moe_router_pre_softmax,
            num_groups=self.config.moe_router_num_groups,
            group_topk=self.config.moe_router_group_topk,
            scaling_factor=self.config.moe_router_topk_scaling_factor,
            score_function=self.score_function,
            expert_bias=self.expert_bias,
            use_hash_routing=self.use_hash_routing,
            hash_table=getattr(self, "tid2eid", None),
            input_ids=input_ids,
        )

    def _loss_stats(self, logits, padding_mask):
        """Which losses apply (``router.py:232-236,320-325``) and their sums,
        from one pass over the logits (``router_loss_stats``)."""
        training = self.training and torch.is_grad_enabled()
        want_z = bool(self.config.moe_z_loss_coeff) and training
        want_aux = (training and not self.use_hash_routing
                    and self.config.moe_aux_loss_coeff > 0.0)
        stats = None
        if want_z or want_aux:
            stats = ops.router_loss_stats(logits, self.topk, self.score_function, padding_mask,
                                          aux=want_aux, z=want_z)
        return want_z, want_aux, stats

    def _finish_routing(self, probs, routing_map, want_aux, stats, padding_mask,
                        accumulate_tokens_per_expert):
        """Aux loss and expert-bias token counts (``router.py:319-354``)."""
        if want_aux:
            probs = self._apply_aux_loss(probs, stats[0], stats[1])
        if self.enable_expert_bias and accumulate_tokens_per_expert and torch.is_grad_enabled():
            with torch.no_grad():
                counts = mask_padding_tokens(routing_map, padding_mask).sum(dim=0).to(torch.float32)
                if not hasattr(self, "local_tokens_per_expert"):
                    self.register_buffer("local_tokens_per_expert", torch.zeros_like(counts),
                                         persistent=False)
                self.local_tokens_per_expert.add_(counts)
        return probs

    def routing(self, logits, input_ids=None, padding_mask=None,
                accumulate_tokens_per_expert: bool = True):
        logits = logits.view(-1, self.config.num_moe_experts)
        input_ids = input_ids.view(-1) if input_ids is not None else None
        if self.use_hash_routing and input_ids is None:
            raise ValueError("Hash routing requires input_ids.")
        # One pass over the logits for both losses (router.py:299, 319-334).
        want_z, want_aux, stats = self._loss_stats(logits, padding_mask)
        logits = self.apply_z_loss(logits, padding_mask=padding_mask,
                                   z_sum=stats[2] if want_z else None)
        if self.routing_type != "none":
            raise ValueError(f"Unsupported MoE routing type: {self.routing_type}")
        probs, routing_map, expert_indices = ops.topk_softmax_with_capacity(
            logits, self.topk, **self._routing_kwargs(input_ids))
        probs = self._finish_routing(probs, routing_map, want_aux, stats, padding_mask,
                                     accumulate_tokens_per_expert)
        return probs, routing_map, expert_indices

    def _can_fuse_gate(self, input) -> bool:
        E = self.config.num_moe_experts
        return (self.routing_type == "none"
                and input.dtype in (torch.bfloat16, torch.float16)
                and self.weight.dtype == input.dtype
                and self.router_dtype(input.dtype) in (input.dtype, torch.float32)
                and E % 32 == 0 and 32 <= E <= 256 and input.shape[-1] % 64 == 0
                and _op_resolves("router_gate_topk"))

    def forward(self, input, input_ids=None, padding_mask=None,
                accumulate_tokens_per_expert: bool = True):
        self._maintain_float32_expert_bias()
        if not self._can_fuse_gate(input):
            logits = self.gating(input)
            probs, routing_map, expert_indices = self.routing(
                logits, input_ids, padding_mask, accumulate_tokens_per_expert)
            return probs, routing_map, expert_indices, logits
        # gating (router.py:84-101) and top-k (router.py:277-317) as one op
        ids = input_ids.view(-1) if input_ids is not None else None
        if self.use_hash_routing and ids is None:
            raise ValueError("Hash routing requires input_ids.")
        if self.weight.device != input.device:
            self.weight.data = self.weight.data.to(device=input.device)
        probs, routing_map, expert_indices, logits = ops.router_gate_topk(
            input, self.weight, self.router_dtype(input.dtype), self.topk,
            **self._routing_kwargs(ids))
        want_z, want_aux, stats = self._loss_stats(logits, padding_mask)
        if want_z:
            probs = MoEAuxLossAutoScaler.apply(
                probs, self._z_loss(logits, padding_mask, stats[2]))
        probs = self._finish_routing(probs, routing_map, want_aux, stats, padding_mask,
                                     accumulate_tokens_per_expert)
        return probs, routing_map, expert_indices, logits.view(*input.shape[:-1], -1)
