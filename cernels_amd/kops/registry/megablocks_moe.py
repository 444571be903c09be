"""megablocks_moe loader (src/kops/registry/megablocks_moe.py:10-24).

Timed path as in the reference: the MoE module's router (megablocks LearnedRouter: bias-free linear,
softmax, top-k, optional p-norm normalisation) and the experts, from the raw hidden state ``x``
[T, H] and the module. Here the router is the fused native router (softmax -> top-k, no
renormalisation; ``moe_normalize_expert_weights`` = 1 maps to its renormalisation) and the experts
run on a packed copy of ``w1`` [E, H, F] / ``w2`` [E, F, H] made on first use and cached on
``moe.experts.mlp``. The activation comes from ``moe.experts.args.activation_fn`` through the
reference loader's name table (gelu -> 0, silu/swish -> 1, relu -> 2; anything unnamed, such as
megablocks' default ``partial(F.gelu, approximate="tanh")``, -> gelu).
"""

import torch

from cernels_amd import ops
from cernels_amd.kops.registry._local import load
from cernels_amd.kops.registry._packed import packed_megablocks

_ACT_IDS = {"gelu": 0, "gelu_new": 0, "gelu_fast": 0, "silu": 1, "swish": 1, "relu": 2}


def act_id_of(args) -> int:
    act_fn = getattr(args, "activation_fn", "gelu")
    name = getattr(act_fn, "__name__", "gelu") if callable(act_fn) else str(act_fn)
    return _ACT_IDS.get(name.lower(), 0)


def kernel(x, moe):
    if moe is None:
        raise RuntimeError("moe module not available (meta device)")
    args = moe.experts.args
    topk = int(args.moe_top_k)
    norm = getattr(args, "moe_normalize_expert_weights", None)
    if norm not in (None, 0, 1, 1.0):
        raise RuntimeError(f"moe_normalize_expert_weights={norm} is not supported (only none or the 1-norm)")
    xf = x.reshape(-1, x.shape[-1]).contiguous()
    with torch.no_grad():
        load("megablocks_moe")  # fail loudly if the native library is missing
        indices, weights = ops.moe_router(xf, moe.router.layer.weight, None, topk, ops.ROUTER_SOFTMAX_TOPK,
                                          renorm=bool(norm))
        packed = packed_megablocks(moe.experts.mlp, ops.MEGABLOCKS_ACTS[act_id_of(args)])
        return ops.moe_experts_packed(xf, packed, indices, weights, topk)
