"""cohere2_moe_experts loader (src/kops/registry/cohere2_moe_experts.py:17-44).

Receives what ``Cohere2MoeExperts.forward`` receives — flat hidden states, top_k_index and
top_k_weights (the router stays outside the op) — plus the experts module for weight storage.
Weight layout: ``gate_up_proj[e]`` is [2F, H], ``down_proj[e]`` is [H, F] (F.linear orientation).
Routing, both grouped GEMMs, the SwiGLU, the routing-weight scale and the combine all run in
the native op. ``kernel`` runs the grouped GEMMs on a packed copy of the module's weights, made
on first use and cached on the module; ``decode_kernel`` streams the weights as stored.
"""

import torch

from cernels_amd import ops
from cernels_amd.kops.registry._local import load
from cernels_amd.kops.registry._packed import packed_experts


def kernel(x, top_k_index, top_k_weights, experts):
    """Prefill: the packed grouped GEMMs on this module's expert weights, packed on first use."""
    if experts is None:
        raise RuntimeError("experts module not available (meta device)")
    with torch.no_grad():
        return ops.moe_experts_packed(
            x.contiguous(),
            packed_experts(experts),  # [E, 2F, H] / [E, H, F], packed once per module
            top_k_index.to(torch.int32).contiguous(),
            top_k_weights.float().contiguous(),
            int(top_k_index.size(1)),
        )


def decode_kernel(x, top_k_index, top_k_weights, experts):
    """Fused gather-GEMV entry point for decode (few tokens) — same contract, two launches."""
    if experts is None:
        raise RuntimeError("experts module not available (meta device)")
    with torch.no_grad():
        return load("cohere2_moe_experts").cohere2_moe_experts_decode(
            x.contiguous(),
            experts.gate_up_proj.data.contiguous(),  # [E, 2F, H]
            experts.down_proj.data.contiguous(),  # [E, H, F]
            top_k_index.to(torch.int32).contiguous(),
            top_k_weights.float().contiguous(),
            int(top_k_index.size(1)),
        )
