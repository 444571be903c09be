"""Per-model expert swaps: replace ``forward`` on every experts instance of a loaded model.

Mirrors src/modeling/swaps.py:13-65 of the reference for its MoE-experts half. ``apply(model,
variant)`` mutates the model in place; ``"stock"`` deletes the instance attribute, restoring the
class method. Variants: ``stock`` → ``custom_prefill`` (prefill entry only) → ``custom``
(prefill + decode entries).

The decode entry handles calls with at most ``DECODE_MAX_TOKENS`` tokens. The reference uses 4
(swaps.py:13); the gfx950 decode GEMV streams each distinct expert once and stays ahead of the
grouped GEMM to well above that, so the threshold here covers the 8-token decode workload too.
"""

from __future__ import annotations

DECODE_MAX_TOKENS = 8


def _experts_fwd(mod, kernel, decode_kernel):
    def fwd(h, idx, w, _m=mod):
        op = decode_kernel if h.size(0) <= DECODE_MAX_TOKENS else kernel
        if op is None:  # this shape's entry point is not enabled in this variant
            return type(_m).forward(_m, h, idx, w)
        return op(h, idx, w, _m)

    return fwd


def _swap_experts(model, cls_name, kernel, decode_kernel):
    """Set (or, with both kernels None, restore) the forward on every ``cls_name`` instance."""
    n = 0
    for mod in model.modules():
        if type(mod).__name__ != cls_name:
            continue
        n += 1
        if "forward" in vars(mod):
            del mod.forward
        if kernel is not None or decode_kernel is not None:
            mod.forward = _experts_fwd(mod, kernel, decode_kernel)
    if not n:
        raise RuntimeError(f"no {cls_name} modules found — wrong model for this swap")
    return n


def north_mini_code(model, variant):
    from cernels_amd.kops.registry.cohere2_moe_experts import decode_kernel, kernel

    return _swap_experts(
        model,
        "Cohere2MoeExperts",
        None if variant == "stock" else kernel,
        decode_kernel if variant == "custom" else None,
    )


def deepseek_ocr_2(model, variant):
    """MoE half of the reference's deepseek_ocr_2 swap (swaps.py:56-65); the SAM rel-pos and
    vision-tower variants of that function are outside the MoE-experts path."""
    from cernels_amd.kops.registry.deepseek_ocr2_moe_experts import decode_kernel, kernel

    moe = variant != "stock"
    return _swap_experts(
        model,
        "DeepseekOcr2TextExperts",
        kernel if moe else None,
        decode_kernel if moe else None,
    )


def qwen3_next(model, variant):
    """Qwen3NextExperts swap (prefill entry; the reference has no qwen3 decode entry)."""
    from cernels_amd.kops.registry.cohere2_moe_experts import decode_kernel, kernel

    return _swap_experts(
        model,
        "Qwen3NextExperts",
        None if variant == "stock" else kernel,
        decode_kernel if variant == "custom" else None,
    )


SWAPS = {
    "north_mini_code": (north_mini_code, ("stock", "custom_prefill", "custom")),
    "deepseek_ocr_2": (deepseek_ocr_2, ("stock", "custom")),
    "qwen3_next": (qwen3_next, ("stock", "custom_prefill", "custom")),
}
