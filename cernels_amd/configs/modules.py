"""Minimal modules with the attribute layout of the transformers MoE blocks the reference uses.

``GptOssMlp``   ~ GptOssMLP:   ``.router`` (GptOssTopKRouter, modeling_gpt_oss.py:117-130) and
                               ``.experts`` (gate_up_proj/down_proj + biases).
``Qwen3NextBlock`` ~ Qwen3NextSparseMoeBlock (modeling_qwen3_next.py:758-797): ``.gate`` router,
                               ``.experts``, ``.shared_expert`` MLP and ``.shared_expert_gate``.
They exist so the drop-in loaders can be exercised without loading model checkpoints; the
loaders accept the transformers modules themselves just as well.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn


class Experts(nn.Module):
    def __init__(self, gate_up_proj, down_proj, gate_up_proj_bias=None, down_proj_bias=None):
        super().__init__()
        self.gate_up_proj = nn.Parameter(gate_up_proj, requires_grad=False)
        self.down_proj = nn.Parameter(down_proj, requires_grad=False)
        self.gate_up_proj_bias = None if gate_up_proj_bias is None else nn.Parameter(gate_up_proj_bias, requires_grad=False)
        self.down_proj_bias = None if down_proj_bias is None else nn.Parameter(down_proj_bias, requires_grad=False)


class GptOssRouter(nn.Module):
    """logits = x Wᵀ + b; top-k of logits; softmax over the k values (in the logits dtype)."""

    def __init__(self, hidden, experts, top_k):
        super().__init__()
        self.top_k, self.num_experts = top_k, experts
        self.weight = nn.Parameter(torch.zeros(experts, hidden), requires_grad=False)
        self.bias = nn.Parameter(torch.zeros(experts), requires_grad=False)

    def forward(self, x):
        logits = F.linear(x, self.weight, self.bias)
        top_v, top_i = torch.topk(logits, self.top_k, dim=-1)
        scores = F.softmax(top_v, dim=1, dtype=top_v.dtype)
        return logits, scores, top_i


class Qwen3NextRouter(nn.Module):
    """softmax(x Wᵀ) in fp32 → top-k → renormalise → logits dtype."""

    def __init__(self, hidden, experts, top_k, norm_topk_prob=True):
        super().__init__()
        self.top_k, self.num_experts, self.norm_topk_prob = top_k, experts, norm_topk_prob
        self.weight = nn.Parameter(torch.zeros(experts, hidden), requires_grad=False)

    def forward(self, x):
        logits = F.linear(x, self.weight)
        probs = F.softmax(logits, dtype=torch.float, dim=-1)
        top_v, top_i = torch.topk(probs, self.top_k, dim=-1)
        if self.norm_topk_prob:
            top_v = top_v / top_v.sum(dim=-1, keepdim=True)
        return logits, top_v.to(logits.dtype), top_i


class DenseMlp(nn.Module):
    """down(silu(gate(x)) * up(x)) — the Qwen3Next shared expert."""

    def __init__(self, hidden, inter):
        super().__init__()
        self.gate_proj = nn.Linear(hidden, inter, bias=False)
        self.up_proj = nn.Linear(hidden, inter, bias=False)
        self.down_proj = nn.Linear(inter, hidden, bias=False)

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class GptOssMlp(nn.Module):
    def __init__(self, router: GptOssRouter, experts: Experts):
        super().__init__()
        self.router, self.experts = router, experts


class Qwen3NextBlock(nn.Module):
    def __init__(self, gate: Qwen3NextRouter, experts: Experts, shared_expert: DenseMlp, shared_expert_gate: nn.Linear):
        super().__init__()
        self.gate, self.experts = gate, experts
        self.shared_expert, self.shared_expert_gate = shared_expert, shared_expert_gate


# ---- megablocks MoE (kernels-community/megablocks, a Hub package absent here): the attribute layout
# the reference loader reads (src/kops/registry/megablocks_moe.py:10-24) and the router it calls.


class MegablocksArgs:
    def __init__(self, hidden, ffn, experts, top_k, activation_fn="gelu", moe_normalize_expert_weights=None):
        self.hidden_size, self.ffn_hidden_size = hidden, ffn
        self.moe_num_experts, self.moe_top_k = experts, top_k
        self.activation_fn = activation_fn
        self.moe_normalize_expert_weights = moe_normalize_expert_weights


class MegablocksRouter(nn.Module):
    """megablocks LearnedRouter: scores = softmax(x Wᵀ) in the input dtype, top-k, optional p-norm."""

    def __init__(self, args: MegablocksArgs):
        super().__init__()
        self.args = args
        self.layer = nn.Linear(args.hidden_size, args.moe_num_experts, bias=False)

    def forward(self, x):
        scores = self.layer(x.view(-1, x.shape[-1])).softmax(dim=-1)
        w, i = torch.topk(scores, self.args.moe_top_k, dim=-1)
        p = self.args.moe_normalize_expert_weights
        if p:
            w = w / torch.norm(w, p=p, dim=-1, keepdim=True)
        return scores, w, i


class MegablocksMlp(nn.Module):
    def __init__(self, w1, w2):
        super().__init__()
        self.w1 = nn.Parameter(w1, requires_grad=False)  # [E, H, F]
        self.w2 = nn.Parameter(w2, requires_grad=False)  # [E, F, H]


class MegablocksExperts(nn.Module):
    def __init__(self, args: MegablocksArgs, mlp: MegablocksMlp):
        super().__init__()
        self.args, self.mlp = args, mlp


class MegablocksMoe(nn.Module):
    def __init__(self, router: MegablocksRouter, experts: MegablocksExperts):
        super().__init__()
        self.router, self.experts = router, experts
