"""Writes the golden fixtures of the MoE-experts path from transformers' own modules.

The reference's op_eager baseline is transformers' experts forward (third-party; the reference
pins transformers>=5.10.2, pyproject.toml:15; this container has 5.15.0). The reference ships no
tests or vectors, so these fixtures are the known answers: tiny seeded modules of each family
are built exactly as the reference's configs build them (params filled N(0, 0.02) after
seeding, src/configs/registry/cohere2_moe_experts.py:54-60), routed by the family's real router
module, and run through the eager experts forward on the CPU in bf16.

Each fixture (safetensors) holds: x, router logits, top_k_index, top_k_weights, the expert
parameters, the expected output ``out``, and ``where_pairs`` — the pair ids p = t*K + k in the
order the eager loop visits them (experts ascending, torch.where over the [K, T] mask).

Run in this container only (the GPU box never imports transformers for tests):
    python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
from pathlib import Path

import torch
import torch.nn.functional as F
from safetensors.torch import save_file

OUT = Path(__file__).resolve().parent


def _fill(module, seed=0):
    torch.manual_seed(seed)
    with torch.no_grad():
        for p in module.parameters():
            p.normal_(0.0, 0.02)
    module.eval()
    return module


def _where_pairs(idx: torch.Tensor, E: int) -> torch.Tensor:
    mask = F.one_hot(idx, num_classes=E).permute(2, 1, 0)
    K = idx.shape[1]
    pairs = []
    for e in range(E):
        kpos, tok = torch.where(mask[e])
        pairs += (tok * K + kpos).tolist()
    return torch.tensor(pairs, dtype=torch.int32)


def _save(name, tensors, meta):
    import transformers

    meta = {**meta, "transformers": transformers.__version__, "torch": torch.__version__}
    save_file({k: v.contiguous() for k, v in tensors.items()}, OUT / f"{name}.safetensors",
              metadata={"meta": json.dumps(meta)})
    print(f"wrote {name}: " + ", ".join(f"{k}{tuple(v.shape)}" for k, v in tensors.items()))


def cohere2(name, T, H, Fi, E, K):
    from transformers.models.cohere2_moe.configuration_cohere2_moe import Cohere2MoeConfig
    from transformers.models.cohere2_moe.modeling_cohere2_moe import Cohere2MoeExperts, Cohere2MoeTopKRouter

    cfg = Cohere2MoeConfig(hidden_size=H, intermediate_size=Fi, num_experts=E, num_experts_per_tok=K,
                           num_shared_experts=0, expert_selection_fn="sigmoid", norm_topk_prob=False,
                           hidden_act="silu")
    cfg._experts_implementation = "eager"
    experts = _fill(Cohere2MoeExperts(cfg).to(torch.bfloat16), 0)
    router = _fill(Cohere2MoeTopKRouter(cfg).to(torch.bfloat16), 2)
    torch.manual_seed(1)
    x = torch.randn(T, H).to(torch.bfloat16)
    with torch.no_grad():
        logits, w, idx = router(x)
        out = experts(x, idx, w)
    _save(name, dict(x=x, logits=logits, top_k_index=idx, top_k_weights=w, gate_up_proj=experts.gate_up_proj.data,
                     down_proj=experts.down_proj.data, out=out, where_pairs=_where_pairs(idx, E)),
          dict(family="cohere2", router="topk_sigmoid", layout="concat", act="silu", T=T, H=H, F=Fi, E=E, K=K))


def deepseek(name, T, H, Fi, E, K):
    from transformers.models.deepseek_ocr2.configuration_deepseek_ocr2 import DeepseekOcr2TextConfig
    from transformers.models.deepseek_ocr2.modeling_deepseek_ocr2 import (
        DeepseekOcr2TextExperts,
        DeepseekOcr2TextTopkRouter,
    )

    cfg = DeepseekOcr2TextConfig(hidden_size=H, moe_intermediate_size=Fi, n_routed_experts=E, num_experts_per_tok=K,
                                 routed_scaling_factor=1.0, topk_method="greedy", hidden_act="silu")
    cfg._experts_implementation = "eager"
    experts = _fill(DeepseekOcr2TextExperts(cfg).to(torch.bfloat16), 0)
    router = _fill(DeepseekOcr2TextTopkRouter(cfg).to(torch.bfloat16), 2)
    torch.manual_seed(1)
    x = torch.randn(T, H).to(torch.bfloat16)
    with torch.no_grad():
        logits, w, idx = router(x)
        w = w.to(torch.bfloat16)  # the caller casts to the hidden dtype (config :85)
        out = experts(x, idx, w)
    _save(name, dict(x=x, logits=logits, top_k_index=idx, top_k_weights=w, gate_up_proj=experts.gate_up_proj.data,
                     down_proj=experts.down_proj.data, out=out, where_pairs=_where_pairs(idx, E)),
          dict(family="deepseek", router="softmax_topk", layout="concat", act="silu", T=T, H=H, F=Fi, E=E, K=K))


def qwen3(name, T, H, Fi, E, K):
    from transformers.models.qwen3_next.configuration_qwen3_next import Qwen3NextConfig
    from transformers.models.qwen3_next.modeling_qwen3_next import Qwen3NextExperts, Qwen3NextTopKRouter

    cfg = Qwen3NextConfig(hidden_size=H, moe_intermediate_size=Fi, shared_expert_intermediate_size=Fi,
                          num_experts=E, num_experts_per_tok=K, norm_topk_prob=True)
    cfg._experts_implementation = "eager"
    experts = _fill(Qwen3NextExperts(cfg).to(torch.bfloat16), 0)
    router = _fill(Qwen3NextTopKRouter(cfg).to(torch.bfloat16), 2)
    torch.manual_seed(1)
    x = torch.randn(T, H).to(torch.bfloat16)
    with torch.no_grad():
        logits, w, idx = router(x)
        out = experts(x, idx, w)
    _save(name, dict(x=x, logits=logits, top_k_index=idx, top_k_weights=w, gate_up_proj=experts.gate_up_proj.data,
                     down_proj=experts.down_proj.data, out=out, where_pairs=_where_pairs(idx, E)),
          dict(family="qwen3", router="softmax_topk_renorm", layout="concat", act="silu", T=T, H=H, F=Fi, E=E, K=K))


def gpt_oss(name, T, H, Fi, E, K):
    from transformers.models.gpt_oss.configuration_gpt_oss import GptOssConfig
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssExperts, GptOssTopKRouter

    cfg = GptOssConfig(hidden_size=H, intermediate_size=Fi, num_local_experts=E, num_experts_per_tok=K)
    cfg._experts_implementation = "eager"
    experts = _fill(GptOssExperts(cfg).to(torch.bfloat16), 0)
    router = _fill(GptOssTopKRouter(cfg).to(torch.bfloat16), 2)
    torch.manual_seed(1)
    # scale x so some gate/up pre-activations cross the +-7 clamp
    x = (torch.randn(T, H) * 4.0).to(torch.bfloat16)
    with torch.no_grad():
        logits, w, idx = router(x)
        out = experts(x, idx, w)
    _save(name, dict(x=x, logits=logits, top_k_index=idx, top_k_weights=w, gate_up_proj=experts.gate_up_proj.data,
                     gate_up_proj_bias=experts.gate_up_proj_bias.data, down_proj=experts.down_proj.data,
                     down_proj_bias=experts.down_proj_bias.data, out=out, where_pairs=_where_pairs(idx, E)),
          dict(family="gpt_oss", router="topk_softmax", layout="interleaved", act="gptoss", T=T, H=H, F=Fi, E=E,
               K=K))


if __name__ == "__main__":
    cohere2("cohere2_t16", T=16, H=64, Fi=64, E=8, K=2)
    cohere2("cohere2_t1", T=1, H=64, Fi=64, E=16, K=8)
    deepseek("deepseek_t12", T=12, H=64, Fi=64, E=8, K=3)
    qwen3("qwen3_t10", T=10, H=64, Fi=64, E=16, K=4)
    gpt_oss("gpt_oss_t9", T=9, H=64, Fi=64, E=4, K=2)
