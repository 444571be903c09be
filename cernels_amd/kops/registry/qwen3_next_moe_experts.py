"""qwen3_next_moe_experts loader (src/kops/registry/qwen3_next_moe_experts.py:21-45).

Everything here is in the timed path; only the hidden state and the
``Qwen3NextSparseMoeBlock``-shaped module come from the caller:
  - router (linear + fp32 softmax + top-k + renorm), the block's own ``gate``;
  - native op: routing + per-expert SwiGLU grouped GEMMs + combine, on a packed copy of the
    expert weights made on first use and cached on the module;
  - the always-on shared expert, ``sigmoid(shared_expert_gate(x)) * shared_expert(x)``, added on top.
Layout: ``gate_up_proj[e]`` is [2F, H], ``down_proj[e]`` is [H, F].
"""

import torch

from cernels_amd import ops
from cernels_amd.kops.registry._local import load
from cernels_amd.kops.registry._packed import packed_experts


def kernel(x, block):
    if block is None:
        raise RuntimeError("block module not available (meta device)")
    bsz, seqlen, hidden = x.shape
    xf = x.reshape(-1, hidden).contiguous()
    with torch.no_grad():
        _logits, scores, indices = block.gate(xf)
        e = block.experts
        load("qwen3_next_moe_experts")  # fail loudly if the native library is missing
        routed = ops.moe_experts_packed(
            xf,
            packed_experts(e),  # [E, 2F, H] / [E, H, F], packed once per module
            indices.to(torch.int32).contiguous(),
            scores.float().contiguous(),
            int(block.gate.top_k),
        )
        shared = block.shared_expert(xf)
        shared = torch.sigmoid(block.shared_expert_gate(xf)) * shared
        out = routed + shared
    return out.reshape(bsz, seqlen, hidden)
