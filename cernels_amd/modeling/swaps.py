"""Instance-level expert swaps: route a loaded model's experts modules through this library.

Contract kept from the reference (src/modeling/swaps.py:20-53): an experts module is called as
``module(hidden, top_k_index, top_k_weights)``; a swapped module instead calls
``op(hidden, top_k_index, top_k_weights, module)`` where ``op`` is a registry loader's
``kernel`` (prefill) or ``decode_kernel`` (few tokens). ``apply(model, variant)`` edits the
model in place and ``"stock"`` restores the class forward. Variants per model are listed in
``SWAPS`` in sweep order, stock first. Only the MoE-experts part of the reference's swaps is
here; its SAM rel-pos and vision-tower variants are other kernels.

Decode dispatch: with the decode entry enabled (variant ``custom``), a call uses the decode GEMV
whenever the GEMV takes it (at most ``DECODE_MAX_TOKENS`` tokens and ``DECODE_MAX_PAIRS`` routed
(token, slot) pairs, the limits of ``cernels_moe_experts_decode``), else the prefill GEMM. Without it
(``custom_prefill``) the reference's switch stays: calls of at most ``REFERENCE_DECODE_TOKENS`` tokens
run the module's own forward and every longer call the prefill op (src/modeling/swaps.py:13,20-27), so a
custom_prefill measurement means what the reference's does. The gfx950 GEMV streams every distinct
selected expert once, so up to its limits it is the faster entry: measured through the ops with the weights rotated over three copies, 66 against
98 us at 16 tokens and 95 against 109 us at 32 on the deepseek-v2-lite expert shapes (k=6), 135
against 166 us and 183 against 212 us on the 30B-A3B shapes (k=8).
"""

from __future__ import annotations

from dataclasses import dataclass
from importlib import import_module

DECODE_MAX_TOKENS = 64   # cernels_moe_decode_max_tokens()
DECODE_MAX_PAIRS = 256   # cernels_moe_decode_max_pairs()
REFERENCE_DECODE_TOKENS = 4  # the reference's decode switch (src/modeling/swaps.py:13)


def use_decode(tokens: int, top_k: int) -> bool:
    """Whether a call of ``tokens`` tokens with ``top_k`` slots each goes to the decode GEMV."""
    return tokens <= DECODE_MAX_TOKENS and tokens * top_k <= DECODE_MAX_PAIRS

_REG = "cernels_amd.kops.registry."


@dataclass(frozen=True)
class ExpertSwap:
    """Which experts class to patch and which loader module supplies ``kernel``/``decode_kernel``."""

    experts_class: str
    loader: str
    variants: tuple[str, ...]


SWAP_TABLE = {
    "north_mini_code": ExpertSwap("Cohere2MoeExperts", "cohere2_moe_experts", ("stock", "custom_prefill", "custom")),
    "deepseek_ocr_2": ExpertSwap("DeepseekOcr2TextExperts", "deepseek_ocr2_moe_experts", ("stock", "custom")),
    # Qwen3NextExperts has the concat layout and plain SwiGLU of the cohere2 op.
    "qwen3_next": ExpertSwap("Qwen3NextExperts", "cohere2_moe_experts", ("stock", "custom_prefill", "custom")),
}


def entry_points(model_name: str, variant: str):
    """(prefill op, decode op) that ``variant`` enables; ``None`` keeps the module's own forward."""
    spec = SWAP_TABLE[model_name]
    if variant not in spec.variants:
        raise KeyError(f"{model_name}: unknown variant {variant!r}; known: {spec.variants}")
    if variant == "stock":
        return None, None
    loader = import_module(_REG + spec.loader)
    decode_on = variant == "custom"
    return loader.kernel, (loader.decode_kernel if decode_on else None)


def _dispatching_forward(module, prefill_op, decode_op):
    stock = type(module).forward

    def forward(hidden, top_k_index, top_k_weights):
        tokens = hidden.size(0)
        if decode_op is not None:
            op = decode_op if use_decode(tokens, top_k_index.size(-1)) else prefill_op
        else:
            op = None if tokens <= REFERENCE_DECODE_TOKENS else prefill_op
        if op is None:
            return stock(module, hidden, top_k_index, top_k_weights)
        return op(hidden, top_k_index, top_k_weights, module)

    return forward


def install(model, experts_class: str, prefill_op, decode_op) -> int:
    """Patch (or, with both ops None, restore) ``forward`` on every ``experts_class`` instance.

    Returns the number of modules touched; raises if the model has none.
    """
    targets = [m for m in model.modules() if type(m).__name__ == experts_class]
    if not targets:
        raise RuntimeError(f"no {experts_class} modules in this model; wrong swap for it")
    for m in targets:
        vars(m).pop("forward", None)
        if prefill_op is not None or decode_op is not None:
            m.forward = _dispatching_forward(m, prefill_op, decode_op)
    return len(targets)


def apply(model, model_name: str, variant: str) -> int:
    prefill_op, decode_op = entry_points(model_name, variant)
    return install(model, SWAP_TABLE[model_name].experts_class, prefill_op, decode_op)


def _model_swap(model_name: str):
    def swap(model, variant):
        return apply(model, model_name, variant)

    swap.__name__ = model_name
    return swap


# name -> (apply(model, variant), variants), the shape of the reference's SWAPS table.
SWAPS = {name: (_model_swap(name), spec.variants) for name, spec in SWAP_TABLE.items()}
north_mini_code = SWAPS["north_mini_code"][0]
deepseek_ocr_2 = SWAPS["deepseek_ocr_2"][0]
qwen3_next = SWAPS["qwen3_next"][0]
