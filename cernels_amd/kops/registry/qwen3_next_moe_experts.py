"""qwen3_next_moe_experts loader (src/kops/registry/qwen3_next_moe_experts.py:21-45).

Everything here is in the timed path; only the hidden state and the
``Qwen3NextSparseMoeBlock``-shaped module come from the caller. The reference runs the block's
router, the experts op, then the always-on shared expert ``sigmoid(shared_expert_gate(x)) *
shared_expert(x)`` and an add, in torch (:28-43). Here two native calls do all of it:
  - the fused router (cernels_moe_router) computes the routing logits and the shared-expert gate
    logit in one GEMM (the gate is the router weight's last row), picks softmax → top-k → renorm,
    and appends S slots per token for the shared expert, weighted bf16(sigmoid(gate logit));
  - the packed experts op runs the routed experts and the shared expert (packed as experts
    E..E+S-1) in the same grouped GEMMs, and its combine sums the K + S rows of each token in fp32
    and rounds once.
Weights are packed on first use and cached on the block. Layout: ``gate_up_proj[e]`` is [2F, H],
``down_proj[e]`` is [H, F].
"""

import torch

from cernels_amd import ops
from cernels_amd.kops.registry._local import load
from cernels_amd.kops.registry._packed import packed_block


def kernel(x, block):
    if block is None:
        raise RuntimeError("block module not available (meta device)")
    bsz, seqlen, hidden = x.shape
    xf = x.reshape(-1, hidden).contiguous()
    with torch.no_grad():
        load("qwen3_next_moe_experts")  # fail loudly if the native library is missing
        gate = block.gate  # Qwen3NextTopKRouter semantics (modeling_qwen3_next.py:766-775), fused
        packed, router_w, S = packed_block(block)
        indices, scores = ops.moe_router(xf, router_w, None, int(gate.top_k), ops.ROUTER_SOFTMAX_TOPK,
                                         renorm=bool(getattr(gate, "norm_topk_prob", True)), shared_slots=S)
        out = ops.moe_experts_packed(xf, packed, indices, scores, int(gate.top_k) + S)
    return out.reshape(bsz, seqlen, hidden)
