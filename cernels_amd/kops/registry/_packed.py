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


def invalidate(experts) -> None:
    """Forget the packed copy (needed after writes through ``param.data``)."""
    if hasattr(experts, _ATTR):
        delattr(experts, _ATTR)


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
