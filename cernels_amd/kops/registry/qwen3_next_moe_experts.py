"""qwen3_next_moe_experts loader (src/kops/registry/qwen3_next_moe_experts.py:21-45).

Everything here is in the timed path; only the hidden state and the
``Qwen3NextSparseMoeBlock``-shaped module come from the caller:
  - router (linear + fp32 softmax + top-k + renorm) on the block's ``gate`` weight, as one fused
    native kernel (cernels_moe_router);
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
        load("qwen3_next_moe_experts")  # fail loudly if the native library is missing
        gate = block.gate  # Qwen3NextTopKRouter semantics (modeling_qwen3_next.py:766-775), fused
        indices, scores = ops.moe_router(xf, gate.weight, None, int(gate.top_k), ops.ROUTER_SOFTMAX_TOPK,
                                         renorm=bool(getattr(gate, "norm_topk_prob", True)))
        routed = ops.moe_experts_packed(
            xf,
            packed_experts(block.experts),  # [E, 2F, H] / [E, H, F], packed once per module
            indices,
            scores,
            int(gate.top_k),
        )
        shared = block.shared_expert(xf)
        shared = torch.sigmoid(block.shared_expert_gate(xf)) * shared
        out = routed + shared
    return out.reshape(bsz, seqlen, hidden)
