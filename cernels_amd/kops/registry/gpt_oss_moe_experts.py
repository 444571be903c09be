"""gpt_oss_moe_experts loader (src/kops/registry/gpt_oss_moe_experts.py:14-47).

The router (linear + top-k + softmax) runs here, in the timed path; only the hidden state and
the ``GptOssMLP``-shaped module come from the caller. The native op does the routing, both
grouped GEMMs with biases and the clamped SwiGLU. Layout: ``gate_up_proj[e]`` is [H, 2F] with
interleaved gate/up columns, ``down_proj[e]`` is [F, H].
"""

import torch

from cernels_amd.kops.registry._local import load


def _weights(e):
    # Expert weights + fp32 bias casts, done once per module (the op consumes fp32 biases and
    # these tensors never change), as the reference caches them (:14-26).
    w = getattr(e, "_kops_weights", None)
    if w is None:
        w = (
            e.gate_up_proj.data.contiguous(),
            e.gate_up_proj_bias.data.float().contiguous(),
            e.down_proj.data.contiguous(),
            e.down_proj_bias.data.float().contiguous(),
        )
        e._kops_weights = w
    return w


def kernel(x, mlp):
    if mlp is None:
        raise RuntimeError("mlp module not available (meta device)")
    bsz, seqlen, hidden = x.shape
    xf = x.reshape(-1, hidden).contiguous()
    with torch.no_grad():
        _logits, scores, indices = mlp.router(xf)  # timed router (same code as the baseline)
        gate_up, gate_up_bias, down, down_bias = _weights(mlp.experts)
        out = load("gpt_oss_moe_experts").gpt_oss_moe_experts(
            xf,
            gate_up,
            gate_up_bias,
            down,
            down_bias,
            indices.to(torch.int32).contiguous(),
            scores.float().contiguous(),
            mlp.router.top_k,
        )
    return out.reshape(bsz, seqlen, hidden)
