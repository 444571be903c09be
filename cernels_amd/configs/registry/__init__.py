"""The registry: every benchmarkable MoE-experts workload, keyed by name.

Two families:

* the five BASELINE workloads (experts only, routing precomputed on the CPU, seeded):
  ``deepseek_v2_lite_decode_t8`` (cfg 1), ``deepseek_v2_lite_prefill`` (cfg 2),
  ``a3b_30b_prefill`` / ``a3b_30b_decode`` (cfg 3), ``gpt_oss_20b_experts`` (cfg 4),
  ``qwen3_next_zipf`` (cfg 5);
* the reference's own config names and routing (src/configs/registry/*_moe_experts.py):
  ``cohere2_moe_experts[_decode]`` (top-k of logits → sigmoid, no renorm),
  ``deepseek_ocr2_moe_experts[_decode]`` (softmax → top-k, scale 1.0, no renorm),
  ``gpt_oss_moe_experts`` (router inside the op call) and ``qwen3_next_moe_experts`` (router and
  shared expert inside the op call).
"""

from __future__ import annotations

import weakref
from types import SimpleNamespace

import torch
from torch import nn

from cernels_amd.configs.base import Config
from cernels_amd.configs.modules import (DenseMlp, Experts, GptOssMlp, GptOssRouter, MegablocksArgs, MegablocksExperts,
                                         MegablocksMlp, MegablocksMoe, MegablocksRouter, Qwen3NextBlock,
                                         Qwen3NextRouter)
from cernels_amd.configs.synth import (
    ACT_GPTOSS,
    INPUT_SEED,
    LAYOUT_INTERLEAVED,
    ROUTER_SOFTMAX_TOPK,
    ROUTER_SOFTMAX_TOPK_RENORM,
    ROUTER_TOPK_SIGMOID,
    ROUTER_TOPK_SOFTMAX,
    WEIGHT_SEED,
    WEIGHT_STD,
    MoeShape,
    make_inputs,
    make_weights,
)
from cernels_amd.kops.registry import cohere2_moe_experts as _cohere2
from cernels_amd.kops.registry import deepseek_ocr2_moe_experts as _deepseek
from cernels_amd.kops.registry import gpt_oss_moe_experts as _gpt_oss
from cernels_amd.kops.registry import megablocks_moe as _megablocks
from cernels_amd.kops.registry import qwen3_next_moe_experts as _qwen3

_DS = dict(hidden=1280, ffn=896, experts=64, top_k=6)
_A3B = dict(hidden=2048, ffn=768, experts=128, top_k=8)
_GPTOSS = dict(hidden=2880, ffn=2880, experts=32, top_k=4, layout=LAYOUT_INTERLEAVED, act=ACT_GPTOSS, bias=True,
               router=ROUTER_TOPK_SOFTMAX)
_QWEN = dict(hidden=2048, ffn=512, experts=512, top_k=10)

# BASELINE.json configs, in order.
BASELINE_SHAPES: dict[str, MoeShape] = {
    s.name: s
    for s in (
        MoeShape("deepseek_v2_lite_decode_t8", tokens=8, decode=True, **_DS),
        MoeShape("deepseek_v2_lite_prefill", tokens=2048, **_DS),
        MoeShape("a3b_30b_prefill", tokens=2048, **_A3B),
        MoeShape("a3b_30b_decode", tokens=1, decode=True, **_A3B),
        MoeShape("gpt_oss_20b_experts", tokens=4096, **_GPTOSS),
        MoeShape("qwen3_next_zipf", tokens=4096, zipf_s=1.2, **_QWEN),
    )
}
BASELINE_ORDER = list(BASELINE_SHAPES)
# The bench headline: BASELINE.json's metric names no config, so the largest workload that fits one GPU
# (configs[3], 815 GFLOP per step).
HEADLINE = "gpt_oss_20b_experts"

# The reference's configs (routing as there).
REFERENCE_SHAPES: dict[str, MoeShape] = {
    s.name: s
    for s in (
        MoeShape("cohere2_moe_experts", tokens=2048, router=ROUTER_TOPK_SIGMOID, **_A3B),
        MoeShape("cohere2_moe_experts_decode", tokens=1, router=ROUTER_TOPK_SIGMOID, decode=True, **_A3B),
        MoeShape("deepseek_ocr2_moe_experts", tokens=2048, router=ROUTER_SOFTMAX_TOPK, **_DS),
        MoeShape("deepseek_ocr2_moe_experts_decode", tokens=1, router=ROUTER_SOFTMAX_TOPK, decode=True, **_DS),
        MoeShape("gpt_oss_moe_experts", tokens=4096, **_GPTOSS),
        MoeShape("qwen3_next_moe_experts", tokens=4096, router=ROUTER_SOFTMAX_TOPK_RENORM, **_QWEN),
    )
}


# stand-in module -> the transformers module built on its tensors (the op_eager baseline)
_OP_EAGER: weakref.WeakKeyDictionary = weakref.WeakKeyDictionary()


def op_eager_module(cfg: Config, standin: nn.Module) -> nn.Module:
    """The transformers module a reference config calls as its op_eager baseline
    (src/configs/registry/cohere2_moe_experts.py:99-104, deepseek_ocr2_moe_experts.py:100-105,
    gpt_oss_moe_experts.py:55-62, qwen3_next_moe_experts.py:66-74): built from its transformers
    config class at the config's shape, with the stand-in's own parameter tensors loaded (so the
    baseline and the drop-in loader compute on identical weights), eager experts dispatch. Built once
    per stand-in."""
    mod = _OP_EAGER.get(standin)
    if mod is not None:
        return mod
    s = cfg.shape
    if isinstance(cfg, GptOssConfig):
        from transformers import GptOssConfig as TC
        from transformers.models.gpt_oss.modeling_gpt_oss import GptOssMLP as cls
        tc = TC(hidden_size=s.hidden, intermediate_size=s.ffn, num_local_experts=s.experts,
                num_experts_per_tok=s.top_k)
    elif isinstance(cfg, Qwen3NextConfig):
        from transformers import Qwen3NextConfig as TC
        from transformers.models.qwen3_next.modeling_qwen3_next import Qwen3NextSparseMoeBlock as cls
        tc = TC(hidden_size=s.hidden, moe_intermediate_size=s.ffn, num_experts=s.experts,
                num_experts_per_tok=s.top_k, shared_expert_intermediate_size=cfg.shared_ffn,
                norm_topk_prob=True, hidden_act="silu")
    elif s.layout == LAYOUT_INTERLEAVED:  # experts-level gpt-oss
        from transformers import GptOssConfig as TC
        from transformers.models.gpt_oss.modeling_gpt_oss import GptOssExperts as cls
        tc = TC(hidden_size=s.hidden, intermediate_size=s.ffn, num_local_experts=s.experts,
                num_experts_per_tok=s.top_k)
    elif s.name.startswith("deepseek"):
        from transformers.models.deepseek_ocr2.modeling_deepseek_ocr2 import DeepseekOcr2TextExperts as cls
        tc = SimpleNamespace(num_experts=s.experts, hidden_size=s.hidden, moe_intermediate_size=s.ffn,
                             hidden_act="silu")
    else:  # the cohere2 experts (the same forward serves the BASELINE experts-level shapes)
        from transformers.models.cohere2_moe.configuration_cohere2_moe import Cohere2MoeConfig as TC
        from transformers.models.cohere2_moe.modeling_cohere2_moe import Cohere2MoeExperts as cls
        tc = TC(hidden_size=s.hidden, intermediate_size=s.ffn, num_experts=s.experts,
                num_experts_per_tok=s.top_k, num_shared_experts=0, expert_selection_fn="sigmoid",
                norm_topk_prob=False, hidden_act="silu")
    tc._experts_implementation = "eager"
    dev = next(standin.parameters()).device
    with torch.device(dev):
        mod = cls(tc)
    mod.load_state_dict({k: v for k, v in standin.state_dict().items() if v is not None}, strict=True)
    mod = mod.to(dtype=cfg.dtype).eval().requires_grad_(False)
    _OP_EAGER[standin] = mod
    return mod


def experts_module(shape: MoeShape, device) -> Experts:
    w = make_weights(shape).to(device)
    return Experts(w.gate_up_proj, w.down_proj, w.gate_up_proj_bias, w.down_proj_bias)


class ExpertsConfig(Config):
    """Experts-level workload: inputs are (x [T,H], top_k_index, top_k_weights, experts)."""

    def __init__(self, shape: MoeShape, custom=None):
        self.shape = shape
        self.name = shape.name
        self.op = f"routed MoE experts T={shape.tokens} H={shape.hidden} F={shape.ffn} E={shape.experts} k={shape.top_k}"
        self.custom = custom

    def baseline(self, x, top_k_index, top_k_weights, experts):
        """op_eager: the transformers experts module on the same tensors."""
        return op_eager_module(self, experts)(x, top_k_index, top_k_weights)

    def inputs(self, device, dtype=torch.bfloat16):
        if str(device) == "meta":
            s = self.shape
            return (torch.empty(s.tokens, s.hidden, device=device, dtype=dtype),
                    torch.zeros(s.tokens, s.top_k, device=device, dtype=torch.int64),
                    torch.empty(s.tokens, s.top_k, device=device, dtype=dtype), None)
        inp = make_inputs(self.shape).to(device)
        return inp.x, inp.top_k_index, inp.top_k_weights, experts_module(self.shape, device)


def _seeded_normal_(module: nn.Module, seed: int = WEIGHT_SEED + 7) -> None:
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in module.parameters():
            p.copy_((torch.randn(p.shape, generator=g) * WEIGHT_STD).to(p.dtype))


class GptOssConfig(Config):
    """Module-level gpt-oss workload (src/configs/registry/gpt_oss_moe_experts.py:23-75)."""

    def __init__(self, shape: MoeShape):
        self.shape, self.name = shape, shape.name
        self.op = "GptOssMLP-shaped (router + clamped-SwiGLU grouped experts)"
        self.custom = staticmethod(_gpt_oss.kernel).__func__

    def baseline(self, x, mlp):
        """op_eager: transformers' GptOssMLP (router + experts) on the same tensors."""
        return op_eager_module(self, mlp)(x)

    def inputs(self, device, dtype=torch.bfloat16):
        s = self.shape
        router = GptOssRouter(s.hidden, s.experts, s.top_k)
        _seeded_normal_(router)
        mlp = GptOssMlp(router, experts_module(s, "cpu")).to(device=device, dtype=dtype)
        g = torch.Generator().manual_seed(INPUT_SEED)
        x = torch.randn((1, s.tokens, s.hidden), generator=g).to(dtype).to(device)
        return x, mlp


class Qwen3NextConfig(Config):
    """Module-level Qwen3-Next workload (src/configs/registry/qwen3_next_moe_experts.py:35-89)."""

    shared_ffn = 512

    def __init__(self, shape: MoeShape):
        self.shape, self.name = shape, shape.name
        self.op = "Qwen3NextSparseMoeBlock-shaped (router + grouped experts + gated shared expert)"
        self.custom = staticmethod(_qwen3.kernel).__func__

    def baseline(self, x, block):
        """op_eager: transformers' Qwen3NextSparseMoeBlock on the same tensors."""
        return op_eager_module(self, block)(x)

    def inputs(self, device, dtype=torch.bfloat16):
        s = self.shape
        gate = Qwen3NextRouter(s.hidden, s.experts, s.top_k)
        shared = DenseMlp(s.hidden, self.shared_ffn)
        sgate = nn.Linear(s.hidden, 1, bias=False)
        for m in (gate, shared, sgate):
            _seeded_normal_(m)
        block = Qwen3NextBlock(gate, experts_module(s, "cpu"), shared, sgate).to(device=device, dtype=dtype)
        g = torch.Generator().manual_seed(INPUT_SEED)
        x = torch.randn((1, s.tokens, s.hidden), generator=g).to(dtype).to(device)
        return x, block


class MegablocksConfig(Config):
    """Module-level megablocks workload (src/configs/registry/megablocks_moe.py:16-78): T=4096, H=2048,
    F=5632, E=8, top-2, no bias, GELU (megablocks' default tanh form), router and experts in the call.
    The reference builds the Hub module (kernels-community/megablocks), absent here; the stand-in has
    its attribute layout and router, with seeded N(0, 0.02) weights."""

    gated = False
    reference_is_hub = True  # the reference's baseline is the Hub kernel, which needs the network
    use_compile = False

    def __init__(self):
        self.name = "megablocks_moe"
        self.shape = MoeShape("megablocks_moe", tokens=4096, hidden=2048, ffn=5632, experts=8, top_k=2)
        self.op = "megablocks MoE (router + non-gated grouped experts)"
        self.custom = staticmethod(_megablocks.kernel).__func__

    def inputs(self, device, dtype=torch.bfloat16):
        s = self.shape
        args = MegablocksArgs(s.hidden, s.ffn, s.experts, s.top_k)
        router = MegablocksRouter(args)
        _seeded_normal_(router)
        g = torch.Generator().manual_seed(WEIGHT_SEED)
        w1 = torch.empty((s.experts, s.hidden, s.ffn), dtype=dtype)
        w2 = torch.empty((s.experts, s.ffn, s.hidden), dtype=dtype)
        for e in range(s.experts):
            w1[e] = (torch.randn((s.hidden, s.ffn), generator=g) * WEIGHT_STD).to(dtype)
        for e in range(s.experts):
            w2[e] = (torch.randn((s.ffn, s.hidden), generator=g) * WEIGHT_STD).to(dtype)
        moe = MegablocksMoe(router, MegablocksExperts(args, MegablocksMlp(w1, w2))).to(device=device, dtype=dtype)
        gx = torch.Generator().manual_seed(INPUT_SEED)
        x = torch.randn((s.tokens, s.hidden), generator=gx).to(dtype).to(device)
        return x, moe


def _make_configs() -> dict[str, Config]:
    cfgs: dict[str, Config] = {}
    for name, s in BASELINE_SHAPES.items():
        if s.layout == LAYOUT_INTERLEAVED:
            cfgs[name] = ExpertsConfig(s, custom=None)  # experts-level gpt-oss: ops.gpt_oss_moe_experts
        else:
            cfgs[name] = ExpertsConfig(s, custom=_cohere2.decode_kernel if s.decode else _cohere2.kernel)
    r = REFERENCE_SHAPES
    cfgs["cohere2_moe_experts"] = ExpertsConfig(r["cohere2_moe_experts"], _cohere2.kernel)
    cfgs["cohere2_moe_experts_decode"] = ExpertsConfig(r["cohere2_moe_experts_decode"], _cohere2.decode_kernel)
    cfgs["deepseek_ocr2_moe_experts"] = ExpertsConfig(r["deepseek_ocr2_moe_experts"], _deepseek.kernel)
    cfgs["deepseek_ocr2_moe_experts_decode"] = ExpertsConfig(r["deepseek_ocr2_moe_experts_decode"], _deepseek.decode_kernel)
    cfgs["gpt_oss_moe_experts"] = GptOssConfig(r["gpt_oss_moe_experts"])
    cfgs["qwen3_next_moe_experts"] = Qwen3NextConfig(r["qwen3_next_moe_experts"])
    cfgs["megablocks_moe"] = MegablocksConfig()
    return cfgs


CONFIGS: dict[str, Config] = _make_configs()
