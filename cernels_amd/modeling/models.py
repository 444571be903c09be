"""Models for the whole-model benchmark (cernels_amd.modeling.main), one builder per swap entry.

The reference loads the real checkpoints by Hub name (src/profiling/registry/north_mini_code.py:
``AutoModelForCausalLM.from_pretrained("CohereLabs/North-Mini-Code-1.0")``). There is no network
here, so a builder takes a local checkpoint directory when one is given and otherwise instantiates
the same transformers architecture with seeded N(0, 0.02) weights on the GPU. Timings depend on the
architecture, not on the weight values. The greedy-match gate then compares stock and swapped runs
of the same random model.

north_mini_code: Cohere2Moe, the shape the reference documents (src/profiling/registry/
north_mini_code.py:1-6 and src/configs/registry/cohere2_moe_experts.py:3-5): 49 decoder layers, layer
0 a dense MLP, layers 1..48 MoE with 128 experts top-8, sigmoid router without renormalisation, no
shared expert, per-expert intermediate 768, hidden 2048, GQA 32 query / 4 key-value heads of 128,
sliding window 4096. Vocabulary 256000 (the Cohere tokenizer). The dense prefix layer's
intermediate size is not stated in the reference; 6144 (3x hidden) is used, and only layer 0 depends
on it.

deepseek_ocr_2: the DeepSeek-V2-lite-style MoE text decoder of DeepseekOcr2 (hidden 1280, 12 layers,
layer 0 dense, 64 routed experts top-6 of intermediate 896, 2 shared experts), run on text tokens
only: the vision tower is built at a token size and never called, so prefill here is the decoder's.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

INIT_STD = 0.02
SEED = 0


@dataclass(frozen=True)
class ModelSpec:
    name: str
    prefill_tokens: int  # the reference's prompt length for this model
    vocab: int
    config: dict = field(default_factory=dict)


NORTH_MINI_CODE = ModelSpec(
    "north_mini_code",
    prefill_tokens=2167,  # README.md:66: "prefill 2167 tokens"
    vocab=256000,
    config=dict(
        vocab_size=256000, hidden_size=2048, num_hidden_layers=49, num_attention_heads=32, num_key_value_heads=4,
        head_dim=128, intermediate_size=768, prefix_dense_intermediate_size=6144, num_experts=128,
        num_experts_per_tok=8, num_shared_experts=0, expert_selection_fn="sigmoid", norm_topk_prob=False,
        sliding_window=4096, first_k_dense_replace=1, max_position_embeddings=8192, hidden_act="silu",
    ),
)

DEEPSEEK_OCR_2 = ModelSpec(
    "deepseek_ocr_2",
    prefill_tokens=1024,
    vocab=129280,
    config=dict(
        vocab_size=129280, hidden_size=1280, intermediate_size=6848, moe_intermediate_size=896,
        num_hidden_layers=12, num_attention_heads=10, num_key_value_heads=10, n_routed_experts=64,
        n_shared_experts=2, num_experts_per_tok=6, first_k_dense_replace=1, max_position_embeddings=8192,
        topk_method="greedy", routed_scaling_factor=1.0, hidden_act="silu",
    ),
)

SPECS = {s.name: s for s in (NORTH_MINI_CODE, DEEPSEEK_OCR_2)}


def make_config(spec: ModelSpec, layers: int | None = None, **overrides):
    """The transformers config of ``spec``; ``layers`` (and ``overrides``) shrink it for tests."""
    kw = dict(spec.config)
    if layers is not None:
        kw["num_hidden_layers"] = int(layers)
    kw.update(overrides)
    if spec.name == "north_mini_code":
        from transformers import Cohere2MoeConfig

        return Cohere2MoeConfig(**kw)
    from transformers.models.deepseek_ocr2.configuration_deepseek_ocr2 import DeepseekOcr2Config

    k = int(kw.pop("first_k_dense_replace", 0))
    kw["mlp_layer_types"] = ["dense" if i < k else "sparse" for i in range(int(kw["num_hidden_layers"]))]

    vision = dict(sam_config=dict(hidden_size=64, output_channels=32, num_hidden_layers=1, num_attention_heads=2,
                                  image_size=64, patch_size=16, global_attn_indexes=[0], window_size=2),
                  encoder_config=dict(hidden_size=64, intermediate_size=128, num_hidden_layers=1,
                                      num_attention_heads=2, num_key_value_heads=2, vocab_size=64))
    return DeepseekOcr2Config(text_config=kw, vision_config=vision)


def _init_random_(model, seed: int = SEED, std: float = INIT_STD) -> None:
    """Seeded N(0, std) weights; norm scales 1 and biases 0, as a freshly initialised model has them."""
    g = torch.Generator(device=next(model.parameters()).device).manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" in name.lower():
                p.fill_(1.0 if name.endswith("weight") else 0.0)
            elif name.endswith("bias"):
                p.zero_()
            else:
                p.normal_(0.0, std, generator=g)


def build(spec: ModelSpec, device="cuda", layers: int | None = None, checkpoint: str | None = None, **overrides):
    """(model in eval mode, bf16, on ``device``). A checkpoint directory is loaded with
    ``from_pretrained``; otherwise the architecture gets seeded random weights."""
    from transformers import AutoModelForCausalLM

    if checkpoint:
        model = AutoModelForCausalLM.from_pretrained(checkpoint, dtype=torch.bfloat16, device_map=str(device))
        return model.eval()
    cfg = make_config(spec, layers, **overrides)
    if spec.name == "north_mini_code":
        from transformers import Cohere2MoeForCausalLM as cls
    else:
        from transformers import DeepseekOcr2ForConditionalGeneration as cls
    with torch.device(device):
        model = cls._from_config(cfg, dtype=torch.bfloat16)
    _init_random_(model)
    return model.eval()


def prompt_ids(spec: ModelSpec, n: int | None = None, device="cuda", vocab: int | None = None) -> dict:
    """Seeded random token ids (the reference tokenises a code prompt; the tokenizer is not here)."""
    n = spec.prefill_tokens if n is None else int(n)
    g = torch.Generator().manual_seed(SEED + 1)
    ids = torch.randint(100, (vocab or spec.vocab) - 1, (1, n), generator=g)
    return {"input_ids": ids.to(device), "attention_mask": torch.ones_like(ids).to(device)}
