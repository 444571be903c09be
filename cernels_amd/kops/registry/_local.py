"""``load(slug)``: the op namespace of one kernel slug.

Mirrors src/kops/registry/_local.py:6-10, which memoises ``kernels.get_local_kernel`` of the
built kernel directory. Here every slug resolves to the same native library; the namespace holds
the slug's ops with the reference names. Loading fails loudly if libcernels_moe.so is missing.
"""

from functools import cache
from types import SimpleNamespace

_OPS = {
    "cohere2_moe_experts": ("cohere2_moe_experts", "cohere2_moe_experts_decode"),
    "deepseek_ocr2_moe_experts": ("deepseek_ocr2_moe_experts", "deepseek_ocr2_moe_experts_decode"),
    "qwen3_next_moe_experts": ("qwen3_next_moe_experts",),
    "gpt_oss_moe_experts": ("gpt_oss_moe_experts",),
    "megablocks_moe": ("megablocks_moe",),
}


@cache
def load(slug: str) -> SimpleNamespace:
    if slug not in _OPS:
        raise KeyError(f"unknown kernel slug {slug!r}; known: {sorted(_OPS)}")
    from cernels_amd import _native, ops

    _native.lib()  # raise now if the native library is absent
    return SimpleNamespace(**{name: getattr(ops, name) for name in _OPS[slug]})
