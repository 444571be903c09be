"""Drop-in loaders (cernels_amd.kops.registry) on module-shaped inputs, against the CPU oracle.

The loaders pack a module's expert weights on first use and cache the packed copy on the module;
a second call reuses it, and an in-place weight update is packed again.
"""

from __future__ import annotations

import pytest
import torch

from helpers import assert_within_tolerance
from oracle import eager as O

pytestmark = pytest.mark.gpu


def _experts(E, H, Fi, layout="concat", bias=False, seed=0, std=0.02):
    from cernels_amd.configs.modules import Experts

    g = torch.Generator().manual_seed(seed)
    if layout == "concat":
        W1, W2 = torch.randn(E, 2 * Fi, H, generator=g) * std, torch.randn(E, H, Fi, generator=g) * std
    else:
        W1, W2 = torch.randn(E, H, 2 * Fi, generator=g) * std, torch.randn(E, Fi, H, generator=g) * std
    b1 = (torch.randn(E, 2 * Fi, generator=g) * std).bfloat16() if bias else None
    b2 = (torch.randn(E, H, generator=g) * std).bfloat16() if bias else None
    return Experts(W1.bfloat16(), W2.bfloat16(), b1, b2)


def test_cohere2_kernel_packs_once_and_repacks_on_update(device):
    from cernels_amd.kops.registry import cohere2_moe_experts as c2

    T, H, Fi, E, K = 300, 256, 128, 8, 3
    ex = _experts(E, H, Fi, seed=1).to(device)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(T, H, generator=g).bfloat16()
    w, idx = torch.topk(torch.softmax(torch.randn(T, E, generator=g), -1), K, -1)
    w = (w / w.sum(-1, keepdim=True)).bfloat16()
    out = c2.kernel(x.to(device), idx.to(device), w.to(device), ex)
    ref = O.experts_fp64(x, idx, w, ex.gate_up_proj.data.cpu(), ex.down_proj.data.cpu())
    assert_within_tolerance(out.cpu(), ref, "cohere2 loader")
    first = ex._cernels_packed[1]
    c2.kernel(x.to(device), idx.to(device), w.to(device), ex)
    assert ex._cernels_packed[1] is first, "packed weights were not reused"
    with torch.no_grad():
        ex.down_proj.mul_(2)  # in-place update of the parameter: must be packed again
    out2 = c2.kernel(x.to(device), idx.to(device), w.to(device), ex)
    assert ex._cernels_packed[1] is not first
    # doubling the down weights doubles every product exactly
    assert torch.equal(out2.float().cpu(), (out.float() * 2).cpu())


def test_gpt_oss_kernel(device):
    from cernels_amd.configs.modules import GptOssMlp, GptOssRouter
    from cernels_amd.kops.registry import gpt_oss_moe_experts as go

    T, H, Fi, E, K = 200, 192, 128, 4, 2
    router = GptOssRouter(H, E, K)
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        router.weight.copy_(torch.randn(E, H, generator=g) * 0.02)
        router.bias.copy_(torch.randn(E, generator=g) * 0.02)
    mlp = GptOssMlp(router, _experts(E, H, Fi, layout="interleaved", bias=True, seed=6, std=0.05)).to(
        device=device, dtype=torch.bfloat16)
    x = torch.randn(1, T, H, generator=g).bfloat16()
    out = go.kernel(x.to(device), mlp)
    from cernels_amd import ops
    xf = x.to(device).reshape(-1, H)
    with torch.no_grad():
        _, mscores, midx = mlp.router(xf)
    idx, scores = ops.moe_router(xf, mlp.router.weight, mlp.router.bias, K, ops.ROUTER_TOPK_SOFTMAX)
    # the fused router agrees with the module's own router except where bf16 logits tie or round apart
    assert (idx.long() == midx).all(dim=1).float().mean() >= 0.95
    e = mlp.experts
    ref = O.experts_fp64(x.reshape(-1, H), idx.cpu(), scores.cpu(), e.gate_up_proj.data.cpu(), e.down_proj.data.cpu(),
                         e.gate_up_proj_bias.data.cpu(), e.down_proj_bias.data.cpu(), layout="interleaved", act="gptoss")
    assert_within_tolerance(out.reshape(-1, H).cpu(), ref, "gpt-oss loader")


@pytest.mark.parametrize("Fs", [64, 96])  # shared intermediate = F, and 1.5 F (two blocks, the last zero-padded)
def test_qwen3_kernel_includes_shared_expert(device, Fs):
    from torch import nn

    from cernels_amd import ops
    from cernels_amd.configs.modules import DenseMlp, Qwen3NextBlock, Qwen3NextRouter
    from cernels_amd.kops.registry import qwen3_next_moe_experts as q3

    T, H, Fi, E, K = 160, 128, 64, 16, 4
    g = torch.Generator().manual_seed(7)
    gate, shared, sgate = Qwen3NextRouter(H, E, K), DenseMlp(H, Fs), nn.Linear(H, 1, bias=False)
    with torch.no_grad():
        for m in (gate, shared, sgate):
            for p in m.parameters():
                p.copy_(torch.randn(p.shape, generator=g) * 0.05)
    block = Qwen3NextBlock(gate, _experts(E, H, Fi, seed=8), shared, sgate).to(device=device, dtype=torch.bfloat16)
    x = torch.randn(1, T, H, generator=g).bfloat16()
    print(f"[qwen3 loader Fs={Fs}]", flush=True)
    out = q3.kernel(x.to(device), block).reshape(-1, H).cpu()
    xf = x.to(device).reshape(-1, H)
    with torch.no_grad():
        _, mscores, midx = block.gate(xf)
    idx, scores = ops.moe_router(xf, block.gate.weight, None, K, ops.ROUTER_SOFTMAX_TOPK)
    # the fused router agrees with the module's own router except where bf16 logits tie or round apart
    assert (idx.long() == midx).all(dim=1).float().mean() >= 0.95
    e, sh = block.experts, block.shared_expert
    routed = O.experts_fp64(x.reshape(-1, H), idx.cpu(), scores.cpu(), e.gate_up_proj.data.cpu(), e.down_proj.data.cpu())
    shared_ref = O.shared_expert_fp64(x.reshape(-1, H), sh.gate_proj.weight.data.cpu(), sh.up_proj.weight.data.cpu(),
                                      sh.down_proj.weight.data.cpu(), block.shared_expert_gate.weight.data.cpu())
    # routed and shared rows are summed in fp32 and rounded once
    assert_within_tolerance(out, routed + shared_ref, "qwen3 loader")
    # the same block called again reuses the packed copy; a changed shared expert is packed again
    pk0 = block._cernels_packed_block[1][0]
    q3.kernel(x.to(device), block)
    assert block._cernels_packed_block[1][0] is pk0
    with torch.no_grad():
        sh.down_proj.weight.mul_(2.0)
    out2 = q3.kernel(x.to(device), block).reshape(-1, H).cpu()
    assert block._cernels_packed_block[1][0] is not pk0
    assert_within_tolerance(out2, routed + 2.0 * shared_ref, "qwen3 loader, shared down doubled")
