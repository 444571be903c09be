"""Per-module cache of expert weights packed for the packed prefill entry.

A module's expert tensors are packed once (``ops.pack_experts``) and the result is kept on the
module, the way the reference's gpt-oss loader keeps fp32 copies of its biases on the module
(src/kops/registry/gpt_oss_moe_experts.py:14-26). The cache is keyed on the storage pointer, the
parameter's in-place version counter and the shape of every source tensor, so a reloaded weight
or an in-place update of the parameter is packed again. A write through ``param.data`` does not
advance the parameter's version counter; after one, drop the cache with ``invalidate(module)``.
The packed copy has the source's element count; the source tensors stay untouched (the decode
entry reads them directly).
"""

from __future__ import annotations

import torch

from cernels_amd import ops

_ATTR = "_cernels_packed"


def _key(params):
    return tuple(None if p is None else (p.data_ptr(), p._version, tuple(p.shape), str(p.device)) for p in params)


def invalidate(module) -> None:
    """Forget the packed copies (needed after writes through ``param.data``)."""
    for attr in (_ATTR, "_cernels_packed_block"):
        if hasattr(module, attr):
            delattr(module, attr)


def packed_experts(experts, *, layout=ops.LAYOUT_CONCAT, act=ops.ACT_SILU, with_bias=False):
    params = (experts.gate_up_proj, experts.down_proj, experts.gate_up_proj_bias if with_bias else None,
              experts.down_proj_bias if with_bias else None)
    key = _key(params) + (layout, act)
    cached = getattr(experts, _ATTR, None)
    if cached is not None and cached[0] == key:
        return cached[1]
    gate_up, down, b1, b2 = (None if p is None else p.data for p in params)
    with torch.no_grad():
        pk = ops.pack_experts(gate_up.contiguous(), down.contiguous(), layout=layout, act=act, gate_up_bias=b1,
                              down_bias=b2)
    setattr(experts, _ATTR, (key, pk))
    return pk


_BLOCK_ATTR = "_cernels_packed_block"


def packed_block(block):
    """Qwen3-Next block: (packed routed + shared experts, router weight [E+1, H], shared slots S).

    The router weight gets the shared-expert gate (``shared_expert_gate.weight``, [1, H]) as its last
    row, so the fused router computes the gate logit with the routing logits. Cached on the block
    with the same keying as ``packed_experts`` (every source tensor of the block).
    """
    e, sh = block.experts, block.shared_expert
    params = (e.gate_up_proj, e.down_proj, sh.gate_proj.weight, sh.up_proj.weight, sh.down_proj.weight,
              block.gate.weight, block.shared_expert_gate.weight)
    key = _key(params)
    cached = getattr(block, _BLOCK_ATTR, None)
    if cached is not None and cached[0] == key:
        return cached[1]
    if getattr(block.shared_expert_gate, "bias", None) is not None:
        raise RuntimeError("shared_expert_gate with a bias is not supported (Qwen3-Next has none)")
    with torch.no_grad():
        pk, S = ops.pack_experts_with_shared(e.gate_up_proj.data, e.down_proj.data, sh.gate_proj.weight.data,
                                             sh.up_proj.weight.data, sh.down_proj.weight.data)
        rw = torch.cat([block.gate.weight.data, block.shared_expert_gate.weight.data], dim=0).contiguous()
    val = (pk, rw, S)
    setattr(block, _BLOCK_ATTR, (key, val))
    return val


def packed_megablocks(mlp, act):
    """megablocks MLP (``w1`` [E, H, F], ``w2`` [E, F, H]) packed for a non-gated activation, cached on
    the MLP module with the same keying as ``packed_experts``."""
    key = _key((mlp.w1, mlp.w2)) + (act,)
    cached = getattr(mlp, _ATTR, None)
    if cached is not None and cached[0] == key:
        return cached[1]
    with torch.no_grad():
        pk = ops.pack_experts_nongated(mlp.w1.data, mlp.w2.data, act)
    setattr(mlp, _ATTR, (key, pk))
    return pk
