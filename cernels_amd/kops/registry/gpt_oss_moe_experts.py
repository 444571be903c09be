"""gpt_oss_moe_experts loader (src/kops/registry/gpt_oss_moe_experts.py:14-47).

The router (linear + bias, top-k of the logits, softmax over the k values) runs here, in the timed
path, as one fused native kernel (cernels_moe_router) reading the module's router weight and bias;
only the hidden state and the ``GptOssMLP``-shaped module come from the caller. The native op then
does the routing, both grouped GEMMs with biases and the clamped SwiGLU, on a packed copy of the
expert weights made on first use and cached on the module. Layout: ``gate_up_proj[e]`` is [H, 2F] with interleaved
gate/up columns, ``down_proj[e]`` is [F, H].
"""

import torch

from cernels_amd import ops
from cernels_amd.kops.registry._local import load
from cernels_amd.kops.registry._packed import packed_experts


def _weights(e):
    # Expert weights packed once per module with fp32 bias copies (the op consumes fp32 biases and
    # these tensors never change), as the reference caches its converted copies (:14-26).
    return packed_experts(e, layout=ops.LAYOUT_INTERLEAVED, act=ops.ACT_GPTOSS, with_bias=True)


def kernel(x, mlp):
    if mlp is None:
        raise RuntimeError("mlp module not available (meta device)")
    bsz, seqlen, hidden = x.shape
    xf = x.reshape(-1, hidden).contiguous()
    with torch.no_grad():
        load("gpt_oss_moe_experts")  # fail loudly if the native library is missing
        r = mlp.router  # GptOssTopKRouter semantics (modeling_gpt_oss.py:126-130), fused
        indices, scores = ops.moe_router(xf, r.weight, r.bias, int(r.top_k), ops.ROUTER_TOPK_SOFTMAX)
        out = ops.moe_experts_packed(xf, _weights(mlp.experts), indices, scores, int(r.top_k))
    return out.reshape(bsz, seqlen, hidden)
