"""Argument checks of the torch-facing ops: a violated contract raises RuntimeError before any
pointer reaches the library (the reference's TORCH_CHECKs, csrc/cohere2_moe_experts.cu:253-257).

CPU: tensors that are not on a GPU are rejected. GPU: every other argument of the packed entry
(device, dtype, contiguity, shape of indices / weights / packed weights / biases / out) is checked
on x's device; none of these calls launches a kernel.
"""

from __future__ import annotations

import pytest
import torch

from cernels_amd import ops


def _packed_cpu(E=2, H=64, F=64):
    gu = torch.zeros(E * 2 * F * H, dtype=torch.bfloat16)
    dn = torch.zeros(E * H * F, dtype=torch.bfloat16)
    return ops.PackedExperts(gu, dn, H, F, E, ops.ACT_SILU, ops.LAYOUT_CONCAT)


def test_packed_entry_rejects_host_tensors():
    pk = _packed_cpu()
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    idx = torch.zeros(4, 2, dtype=torch.int32)
    w = torch.zeros(4, 2, dtype=torch.float32)
    with pytest.raises(RuntimeError, match="x must be"):
        ops.moe_experts_packed(x, pk, idx, w, 2)
    with pytest.raises(RuntimeError, match="packed must come from"):
        ops.moe_experts_packed(x, object(), idx, w, 2)


def test_stored_layout_entry_rejects_host_tensors():
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    W1 = torch.zeros(2, 128, 64, dtype=torch.bfloat16)
    W2 = torch.zeros(2, 64, 64, dtype=torch.bfloat16)
    idx = torch.zeros(4, 2, dtype=torch.int32)
    w = torch.zeros(4, 2, dtype=torch.float32)
    with pytest.raises(RuntimeError, match="CUDA"):
        ops.moe_experts(x, W1, W2, idx, w, 2)


@pytest.mark.gpu
def test_packed_entry_checks_every_argument(device):
    E, H, F, T, K = 2, 64, 64, 4, 2
    g = torch.Generator().manual_seed(0)
    W1 = (torch.randn(E, 2 * F, H, generator=g) * 0.02).bfloat16().to(device)
    W2 = (torch.randn(E, H, F, generator=g) * 0.02).bfloat16().to(device)
    pk = ops.pack_experts(W1, W2)
    x = torch.randn(T, H, generator=g).bfloat16().to(device)
    idx = torch.zeros(T, K, dtype=torch.int32, device=device)
    w = torch.full((T, K), 0.5, dtype=torch.float32, device=device)
    good = ops.moe_experts_packed(x, pk, idx, w, K)  # the valid call works
    torch.cuda.synchronize()
    assert good.shape == (T, H)
    bad = {
        "indices on the host": dict(indices=idx.cpu()),
        "weights on the host": dict(weights=w.cpu()),
        "indices int64": dict(indices=idx.long()),
        "weights bf16": dict(weights=w.bfloat16()),
        "indices not contiguous": dict(indices=torch.zeros(K, T, dtype=torch.int32, device=device).t()),
        "indices wrong shape": dict(indices=torch.zeros(T, K + 1, dtype=torch.int32, device=device)),
        "out on the host": dict(out=torch.empty(T, H, dtype=torch.bfloat16)),
        "out too small": dict(out=torch.empty(T - 1, H, dtype=torch.bfloat16, device=device)),
        "out fp32": dict(out=torch.empty(T, H, dtype=torch.float32, device=device)),
        "out not contiguous": dict(out=torch.empty(H, T, dtype=torch.bfloat16, device=device).t()),
    }
    for what, kw in bad.items():
        args = dict(x=x, packed=pk, indices=idx, weights=w, topk=K) | kw
        with pytest.raises(RuntimeError):
            ops.moe_experts_packed(**args)
        print(f"[checks] rejected: {what}", flush=True)
    host_pk = ops.PackedExperts(pk.gate_up.cpu(), pk.down, pk.H, pk.F, pk.E, pk.act, pk.bias_layout)
    with pytest.raises(RuntimeError, match="packed gate_up"):
        ops.moe_experts_packed(x, host_pk, idx, w, K)
    for what, kw in {"gate_up packed for fewer experts": dict(gate_up=pk.gate_up[: pk.gate_up.numel() // 2]),
                     "down packed for fewer experts": dict(down=pk.down[: pk.down.numel() // 2]),
                     "more experts than packed": dict(E=E + 1)}.items():
        f = dict(gate_up=pk.gate_up, down=pk.down, E=pk.E) | kw
        short_pk = ops.PackedExperts(f["gate_up"], f["down"], pk.H, pk.F, f["E"], pk.act, pk.bias_layout)
        with pytest.raises(RuntimeError, match="packed"):
            ops.moe_experts_packed(x, short_pk, idx, w, K)
        print(f"[checks] rejected: {what}", flush=True)
    bias_pk = ops.PackedExperts(pk.gate_up, pk.down, pk.H, pk.F, pk.E, pk.act, pk.bias_layout,
                                gate_up_bias=torch.zeros(E, 2 * F, device=device, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="biases"):
        ops.moe_experts_packed(x, bias_pk, idx, w, K)
