"""Seeded synthetic MoE-experts workloads.

Every tensor is generated on the CPU with ``torch.Generator().manual_seed(s)`` and only then
copied to the target device, so a CPU checker and the GPU path see bit-identical inputs.
Seed 0 drives the expert parameters, seed 1 drives the hidden states and the routing, which
mirrors the reference harness (src/configs/registry/cohere2_moe_experts.py:54 seeds the module
with 0 and :72 seeds x/routing with 1). The reference draws its tensors on the GPU; these are
drawn on the CPU on purpose, so that routing is computed once, in fp32, and shared.

Weight layouts follow the transformers experts modules the reference wraps:

* ``concat`` (Cohere2Moe / DeepseekOcr2 / Qwen3Next experts): ``gate_up_proj[E, 2F, H]`` with
  rows ``[0, F)`` the gate and ``[F, 2F)`` the up projection, ``down_proj[E, H, F]``
  (``F.linear`` orientation; src/kops/cohere2_moe_experts/csrc/cohere2_moe_experts.cu:5-17).
* ``interleaved`` (gpt-oss): ``gate_up_proj[E, H, 2F]`` with even columns the gate and odd
  columns the up projection, ``down_proj[E, F, H]``, plus ``gate_up_proj_bias[E, 2F]`` and
  ``down_proj_bias[E, H]`` (src/kops/gpt_oss_moe_experts/csrc/gpt_oss_moe_experts.cu:3-20).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, replace

import torch

WEIGHT_SEED = 0
INPUT_SEED = 1
WEIGHT_STD = 0.02

LAYOUT_CONCAT = "concat"
LAYOUT_INTERLEAVED = "interleaved"
ACT_SILU = "silu"
ACT_GPTOSS = "gptoss"

# Routers. Each maps fp32 logits [T, E] to (top_k_index int64 [T, k], top_k_weights bf16 [T, k]).
ROUTER_SOFTMAX_TOPK_RENORM = "softmax_topk_renorm"  # Qwen3NextTopKRouter, norm_topk_prob=True
ROUTER_SOFTMAX_TOPK = "softmax_topk"  # DeepseekOcr2 greedy, routed_scaling_factor=1.0
ROUTER_TOPK_SOFTMAX = "topk_softmax"  # GptOssTopKRouter
ROUTER_TOPK_SIGMOID = "topk_sigmoid"  # Cohere2MoeTopKRouter, sigmoid, no renorm


@dataclass(frozen=True)
class MoeShape:
    """One experts workload: shapes, weight layout, activation, router and routing skew."""

    name: str
    tokens: int
    hidden: int
    ffn: int
    experts: int
    top_k: int
    layout: str = LAYOUT_CONCAT
    act: str = ACT_SILU
    bias: bool = False
    router: str = ROUTER_SOFTMAX_TOPK_RENORM
    zipf_s: float = 0.0  # >0: per-expert logit bias so popularity follows Zipf(s)
    decode: bool = False  # the op entry this workload exercises

    def with_tokens(self, tokens: int, decode: bool | None = None) -> "MoeShape":
        return replace(self, tokens=tokens, decode=self.decode if decode is None else decode)

    @property
    def pairs(self) -> int:
        return self.tokens * self.top_k

    def flops(self) -> float:
        """Algorithmic FLOPs: 2·(T·k)·H·2F for gate_up plus 2·(T·k)·F·H for down."""
        return 6.0 * self.tokens * self.top_k * self.hidden * self.ffn

    def expert_bytes(self) -> int:
        """Bytes of one expert's weights (gate_up + down, bf16, plus biases if any)."""
        b = 3 * self.hidden * self.ffn * 2
        if self.bias:
            b += (2 * self.ffn + self.hidden) * 2
        return b


@dataclass
class MoeWeights:
    """Expert parameters, attribute names as on the transformers experts modules."""

    gate_up_proj: torch.Tensor
    down_proj: torch.Tensor
    gate_up_proj_bias: torch.Tensor | None = None
    down_proj_bias: torch.Tensor | None = None

    def to(self, device) -> "MoeWeights":
        mv = lambda t: None if t is None else t.to(device)  # noqa: E731
        return MoeWeights(mv(self.gate_up_proj), mv(self.down_proj), mv(self.gate_up_proj_bias), mv(self.down_proj_bias))


@dataclass
class MoeInputs:
    x: torch.Tensor  # [T, H] bf16
    top_k_index: torch.Tensor  # [T, k] int64
    top_k_weights: torch.Tensor  # [T, k] bf16
    logits: torch.Tensor  # [T, E] fp32 (router input, kept for router tests)

    def to(self, device) -> "MoeInputs":
        return MoeInputs(self.x.to(device), self.top_k_index.to(device), self.top_k_weights.to(device), self.logits.to(device))


def make_weights(shape: MoeShape, seed: int = WEIGHT_SEED, std: float = WEIGHT_STD) -> MoeWeights:
    """N(0, std) bf16 parameters, drawn expert by expert (bounded host memory at 512 experts)."""
    g = torch.Generator().manual_seed(seed)
    E, H, F = shape.experts, shape.hidden, shape.ffn
    if shape.layout == LAYOUT_CONCAT:
        gu_shape, dn_shape = (2 * F, H), (H, F)
    elif shape.layout == LAYOUT_INTERLEAVED:
        gu_shape, dn_shape = (H, 2 * F), (F, H)
    else:
        raise ValueError(f"unknown layout {shape.layout!r}")
    gate_up = torch.empty((E, *gu_shape), dtype=torch.bfloat16)
    down = torch.empty((E, *dn_shape), dtype=torch.bfloat16)
    for e in range(E):
        gate_up[e] = (torch.randn(gu_shape, generator=g) * std).to(torch.bfloat16)
    for e in range(E):
        down[e] = (torch.randn(dn_shape, generator=g) * std).to(torch.bfloat16)
    gub = db = None
    if shape.bias:
        gub = (torch.randn((E, 2 * F), generator=g) * std).to(torch.bfloat16)
        db = (torch.randn((E, H), generator=g) * std).to(torch.bfloat16)
    return MoeWeights(gate_up, down, gub, db)


def zipf_logit_bias(experts: int, s: float, g: torch.Generator) -> torch.Tensor:
    """b_e = -s·ln(r_e), r a seeded permutation of 1..E: softmax popularity ∝ r_e^-s (Zipf s)."""
    r = torch.randperm(experts, generator=g).to(torch.float64) + 1.0
    return (-s * torch.log(r)).to(torch.float32)


def route(logits: torch.Tensor, top_k: int, router: str) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 logits [T, E] → (int64 index [T, k], bf16 weights [T, k]).

    Restates the transformers routers the reference feeds its op with:
    Qwen3NextTopKRouter (modeling_qwen3_next.py:766-775), DeepseekOcr2TextTopkRouter greedy
    (modeling_deepseek_ocr2.py:1189-1208), GptOssTopKRouter (modeling_gpt_oss.py:126-130) and
    Cohere2MoeTopKRouter sigmoid (modeling_cohere2_moe.py:150-163).
    """
    logits = logits.float()
    if router in (ROUTER_SOFTMAX_TOPK_RENORM, ROUTER_SOFTMAX_TOPK):
        probs = torch.softmax(logits, dim=-1, dtype=torch.float32)
        w, idx = torch.topk(probs, top_k, dim=-1)
        if router == ROUTER_SOFTMAX_TOPK_RENORM:
            w = w / w.sum(dim=-1, keepdim=True)
    elif router == ROUTER_TOPK_SOFTMAX:
        v, idx = torch.topk(logits, top_k, dim=-1)
        w = torch.softmax(v, dim=1, dtype=torch.float32)
    elif router == ROUTER_TOPK_SIGMOID:
        v, idx = torch.topk(logits, top_k, dim=-1)
        w = torch.sigmoid(v)
    else:
        raise ValueError(f"unknown router {router!r}")
    return idx, w.to(torch.bfloat16)


def make_inputs(shape: MoeShape, seed: int = INPUT_SEED) -> MoeInputs:
    """x ~ N(0,1) bf16, router logits ~ N(0,1) fp32 (+ Zipf bias), routed on the CPU."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((shape.tokens, shape.hidden), generator=g).to(torch.bfloat16)
    logits = torch.randn((shape.tokens, shape.experts), generator=g)
    if shape.zipf_s > 0:
        logits = logits + zipf_logit_bias(shape.experts, shape.zipf_s, g)
    idx, w = route(logits, shape.top_k, shape.router)
    return MoeInputs(x, idx, w, logits)


def distinct_experts(top_k_index: torch.Tensor) -> int:
    return int(torch.unique(top_k_index.flatten()).numel())


def weight_bytes_touched(shape: MoeShape, top_k_index: torch.Tensor) -> int:
    """Algorithmic weight bytes: each distinct routed expert's parameters once."""
    return distinct_experts(top_k_index) * shape.expert_bytes()


def activation_bytes(shape: MoeShape) -> int:
    """x read + out written (bf16), index int32 + weight fp32 read."""
    return 2 * shape.tokens * shape.hidden * 2 + shape.pairs * 8


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)


def zipf_expected_max_share(experts: int, s: float) -> float:
    """Share of routing mass on the most popular expert under Zipf(s) (for reporting)."""
    z = sum(r ** -s for r in range(1, experts + 1))
    return 1.0 / z if z > 0 else math.nan
