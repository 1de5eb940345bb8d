"""MoE layer workloads and their seeded synthetic inputs.

The five configurations of the path's benchmark definition: toy (fp32, CPU
sized), Mixtral-, Qwen3-30B-A3B- and DeepSeek-V3-shaped layers and a packed
variable-length stress case. Router logits are supplied directly (the
configurations specify their distribution):

* N(0, 1), fp32, for toy and Mixtral;
* Qwen3: N(0, 1) + b_e with b_e = -1.1 ln(rank_e), rank a seeded permutation
  of 1..E (a Zipf(s=1.1) prior on expert load), fp32;
* DeepSeek-V3: N(0, 1) fp32 logits, sigmoid scores, a small seeded expert
  bias, 8 groups / 4 kept, scaling 2.5; FP8 weights (128x128 block scales);
* varlen: 32 samples of U[64, 4096] tokens, right-padded to a multiple of
  256; a seeded 30% of tokens get +8 on 4 hot experts and 8 dead experts get
  -1e4 (empty segments).

Weights are N(0, 0.02); fc1 is ``[E, H, 2F]`` (gate | up) and fc2 ``[E, F, H]``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    tokens: int
    hidden: int
    experts: int
    topk: int
    ffn: int
    dtype: torch.dtype = torch.bfloat16
    pre_softmax: bool = False
    score_function: str = "softmax"
    num_groups: int | None = None
    group_topk: int | None = None
    scaling_factor: float | None = None
    expert_bias: bool = False
    fp8: bool = False
    shared_ffn: int | None = None
    logits: str = "normal"  # normal | zipf | varlen
    seed: int = 0
    extra: dict = field(default_factory=dict, compare=False, hash=False)

    @property
    def routed_rows(self) -> int:
        return self.tokens * self.topk

    def gemm_flops_fwd_bwd(self) -> float:
        """18 * M * H * F: fc1 (H -> 2F) and fc2 (F -> H), forward + dX + dW."""
        return 18.0 * self.routed_rows * self.hidden * self.ffn

    def permute_bytes(self) -> float:
        """One permute pass: (T + M) * H * b + 12 * T * k."""
        b = torch.finfo(self.dtype).bits // 8
        return (self.tokens + self.routed_rows) * self.hidden * b + 12.0 * self.routed_rows


TOY = Workload("toy", 512, 256, 8, 2, 512, dtype=torch.float32)
MIXTRAL = Workload("mixtral", 8192, 4096, 8, 2, 14336)
QWEN3 = Workload("qwen3_30b_a3b", 16384, 2048, 128, 8, 768, logits="zipf")
DSV3 = Workload("deepseek_v3", 4096, 7168, 256, 8, 2048, score_function="sigmoid",
                num_groups=8, group_topk=4, scaling_factor=2.5, expert_bias=True, fp8=True,
                shared_ffn=2048)
VARLEN = Workload("varlen_stress", 0, 2048, 128, 8, 768, logits="varlen")

WORKLOADS = {w.name: w for w in (TOY, MIXTRAL, QWEN3, DSV3, VARLEN)}


def varlen_lengths(seed: int = 0, samples: int = 32) -> list[int]:
    g = torch.Generator().manual_seed(seed + 17)
    return [int(x) for x in torch.randint(64, 4097, (samples,), generator=g)]


def varlen_tokens(seed: int = 0) -> int:
    total = sum(varlen_lengths(seed))
    return ((total + 255) // 256) * 256


def resolve(w: Workload) -> Workload:
    if w.logits == "varlen" and w.tokens == 0:
        from dataclasses import replace
        return replace(w, tokens=varlen_tokens(w.seed))
    return w


def make_logits(w: Workload, device="cpu") -> torch.Tensor:
    w = resolve(w)
    g = torch.Generator().manual_seed(w.seed)
    logits = torch.randn(w.tokens, w.experts, generator=g)
    if w.logits in ("zipf", "varlen"):
        rank = torch.randperm(w.experts, generator=g).double() + 1.0
        logits += (-1.1 * torch.log(rank)).float()
    if w.logits == "varlen":
        hot = torch.randperm(w.experts, generator=g)[:12]
        hot_tokens = torch.rand(w.tokens, generator=g) < 0.30
        logits[hot_tokens.nonzero().squeeze(1).unsqueeze(1), hot[:4].unsqueeze(0)] += 8.0
        logits[:, hot[4:12]] = -1e4
    return logits.to(device)


def make_expert_bias(w: Workload, device="cpu") -> torch.Tensor | None:
    if not w.expert_bias:
        return None
    g = torch.Generator().manual_seed(w.seed + 3)
    return (torch.randn(w.experts, generator=g) * 0.01).to(device)


def make_weights(w: Workload, device="cpu", std: float = 0.02):
    """(w1 [E, H, 2F], w2 [E, F, H]) in the workload dtype, seeded."""
    w = resolve(w)
    if torch.device(device).type == "cuda":
        g = torch.Generator(device=device).manual_seed(w.seed + 1)
    else:
        g = torch.Generator().manual_seed(w.seed + 1)
    w1 = torch.empty(w.experts, w.hidden, 2 * w.ffn, dtype=torch.float32, device=device)
    w1.normal_(0.0, std, generator=g)
    w2 = torch.empty(w.experts, w.ffn, w.hidden, dtype=torch.float32, device=device)
    w2.normal_(0.0, std, generator=g)
    return w1.to(w.dtype), w2.to(w.dtype)


def make_hidden(w: Workload, device="cpu") -> torch.Tensor:
    w = resolve(w)
    if torch.device(device).type == "cuda":
        g = torch.Generator(device=device).manual_seed(w.seed + 2)
    else:
        g = torch.Generator().manual_seed(w.seed + 2)
    x = torch.empty(w.tokens, w.hidden, dtype=torch.float32, device=device)
    x.normal_(0.0, 1.0, generator=g)
    return x.to(w.dtype)


def make_grad(w: Workload, device="cpu") -> torch.Tensor:
    w = resolve(w)
    if torch.device(device).type == "cuda":
        g = torch.Generator(device=device).manual_seed(w.seed + 4)
    else:
        g = torch.Generator().manual_seed(w.seed + 4)
    d = torch.empty(w.tokens, w.hidden, dtype=torch.float32, device=device)
    d.normal_(0.0, 1.0, generator=g)
    return d.to(w.dtype)


def fp8_blocks(weight: torch.Tensor):
    """[E, R, C] -> (e4m3fn [E, R, C], bf16 scales [E, R/128, C/128]); s = amax / 448."""
    E, R, C = weight.shape
    br, bc = math.ceil(R / 128), math.ceil(C / 128)
    wf = weight.float()
    if R % 128 or C % 128:
        pad = torch.zeros(E, br * 128, bc * 128, device=weight.device)
        pad[:, :R, :C] = wf
        wf_p = pad
    else:
        wf_p = wf
    amax = wf_p.view(E, br, 128, bc, 128).abs().amax(dim=(2, 4))
    scale = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax)).to(torch.bfloat16)
    full = scale.float().repeat_interleave(128, 1).repeat_interleave(128, 2)[:, :R, :C]
    q = (wf / full).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q, scale
