"""megablocks_moe (non-gated experts: act(x W1) W2, gelu/silu/relu) on the GPU against the fp64 oracle.

The reference op's own reference is the megablocks Hub kernel (src/configs/registry/megablocks_moe.py:
reference_is_hub), which is absent here; parity is pinned on oracle.eager.megablocks_fp64, itself
pinned on the CPU (brute force, and silu tied to the golden-pinned gated experts). Bar: the
experts' tolerance, |out - fp64| <= 2e-2 RMS + half a bf16 ulp elementwise; the reference-named op
(packs per call) and the packed entry (packed once) agree bit for bit.
"""

from __future__ import annotations

import random

import pytest
import torch

from helpers import assert_within_tolerance
from oracle import eager as O

pytestmark = pytest.mark.gpu


def _case(seed, T, H, F, E, K, std=0.05, invalid=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).bfloat16()
    w1 = (torch.randn(E, H, F, generator=g) * std).bfloat16()
    w2 = (torch.randn(E, F, H, generator=g) * std).bfloat16()
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).int()
    if invalid:
        pos = torch.randperm(T * K, generator=g)[:invalid]
        idx.view(-1)[pos] = torch.where(torch.arange(invalid) % 2 == 0, torch.tensor(-1), torch.tensor(E)).int()
    wt = torch.rand(T, K, generator=g)
    return x, w1, w2, idx, wt


CASES = [
    # (seed, T, H, F, E, K, act_id, invalid ids)
    (0, 37, 128, 64, 8, 2, 0, 0),
    (1, 300, 256, 192, 16, 4, 1, 0),
    (2, 513, 64, 128, 5, 2, 2, 0),
    (3, 1, 128, 320, 4, 2, 0, 0),
    (4, 1200, 192, 256, 8, 2, 1, 17),
    (5, 90, 320, 64, 3, 1, 2, 3),
]


def _sweep(n=12, seed=20261204):
    """Seeded random legal shapes (H, F any multiple of 64 up to 768, 1-16 experts, top-1..4, 1-700 tokens, each
    activation, a few invalid ids): the same list on every run."""
    r = random.Random(seed)
    out = []
    for i in range(n):
        E = r.randint(1, 16)
        K = r.randint(1, min(E, 4))
        T = r.randint(1, 700)
        out.append((3000 + i, T, 64 * r.randint(1, 12), 64 * r.randint(1, 12), E, K, i % 3,
                    r.randint(0, 3) if T * K > 3 else 0))
    return out


CASES += _sweep()


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"T{c[1]}H{c[2]}F{c[3]}E{c[4]}k{c[5]}a{c[6]}")
def test_megablocks_op_matches_oracle(device, case):
    from cernels_amd import ops

    seed, T, H, F, E, K, act_id, invalid = case
    x, w1, w2, idx, wt = _case(seed, T, H, F, E, K, invalid=invalid)
    print(f"[megablocks {case}]", flush=True)
    d = [t.to(device) for t in (x, w1, w2, idx, wt)]
    out = ops.megablocks_moe(*d, K, act_id)
    ref = O.megablocks_fp64(x, idx, wt, w1, w2, act_id)
    assert_within_tolerance(out.cpu(), ref, f"megablocks act {act_id}")
    # the packed entry on weights packed once gives the same bits
    pk = ops.pack_experts_nongated(d[1], d[2], ops.MEGABLOCKS_ACTS[act_id])
    out2 = ops.moe_experts_packed(d[0], pk, d[3], d[4], K)
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))


def test_megablocks_loader_with_router(device):
    from cernels_amd import ops
    from cernels_amd.configs.modules import (MegablocksArgs, MegablocksExperts, MegablocksMlp, MegablocksMoe,
                                             MegablocksRouter)
    from cernels_amd.kops.registry import megablocks_moe as mb

    T, H, F, E, K = 200, 128, 192, 8, 2
    x, w1, w2, _, _ = _case(9, T, H, F, E, K)
    for act_name, act_id in (("gelu", 0), ("silu", 1), ("relu", 2)):
        args = MegablocksArgs(H, F, E, K, activation_fn=act_name)
        router = MegablocksRouter(args)
        with torch.no_grad():
            router.layer.weight.copy_(torch.randn(E, H, generator=torch.Generator().manual_seed(act_id)) * 0.1)
        moe = MegablocksMoe(router, MegablocksExperts(args, MegablocksMlp(w1.clone(), w2.clone())))
        moe = moe.to(device=device, dtype=torch.bfloat16)
        print(f"[megablocks loader {act_name}]", flush=True)
        xd = x.to(device)
        out = mb.kernel(xd, moe).cpu()
        idx, wts = ops.moe_router(xd, moe.router.layer.weight, None, K, ops.ROUTER_SOFTMAX_TOPK, renorm=False)
        with torch.no_grad():
            _, mw, mi = moe.router(xd)
        # same experts as the module's bf16 softmax -> top-k, except where bf16 probabilities tie
        assert (idx.long().sort(dim=1).values == mi.sort(dim=1).values).all(dim=1).float().mean() >= 0.95
        ref = O.megablocks_fp64(x, idx.cpu(), wts.cpu(), w1, w2, act_id)
        assert_within_tolerance(out, ref, f"megablocks loader {act_name}")
        # packed once: the second call reuses the cache
        pk = moe.experts.mlp._cernels_packed[1]
        mb.kernel(xd, moe)
        assert moe.experts.mlp._cernels_packed[1] is pk


def test_megablocks_full_size(device):
    """The reference's config shape: T=4096, H=2048, F=5632, E=8, top-2, GELU, near-uniform routing."""
    from cernels_amd import ops

    T, H, F, E, K = 4096, 2048, 5632, 8, 2
    print("[megablocks full] generating", flush=True)
    x, w1, w2, idx, wt = _case(21, T, H, F, E, K, std=0.02)
    d = [t.to(device) for t in (x, w1, w2, idx, wt)]
    print("[megablocks full] run", flush=True)
    out = ops.megablocks_moe(*d, K, 0)
    out2 = ops.megablocks_moe(*d, K, 0)
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), "not run-to-run deterministic"
    rows = torch.randperm(T, generator=torch.Generator().manual_seed(0))[:48]
    st = assert_within_tolerance(out.cpu()[rows], O.megablocks_fp64(x[rows], idx[rows], wt[rows], w1, w2, 0),
                                 "megablocks full", strict=True)
    print(f"[megablocks full] max|err|/RMS = {st['ratio']:.4f}", flush=True)
    # linearity in the routing weights: doubled weights give exactly doubled fp32 sums (one rounding)
    out_x2 = ops.megablocks_moe(d[0], d[1], d[2], d[3], 2 * d[4], K, 0)
    assert torch.equal((2 * out.float()).bfloat16().view(torch.int16), out_x2.view(torch.int16))


def test_megablocks_rejects(device):
    from cernels_amd import _native, ops

    x, w1, w2, idx, wt = _case(0, 8, 128, 64, 4, 2)
    d = [t.to(device) for t in (x, w1, w2, idx, wt)]
    with pytest.raises(RuntimeError):
        ops.megablocks_moe(*d, 2, 3)  # act_id outside 0..2
    with pytest.raises(RuntimeError):
        ops.megablocks_moe(d[0], d[1][:, :, :48].contiguous(), d[2][:, :48].contiguous(), d[3], d[4], 2, 0)  # F % 64
    # non-gated activations exist only on the packed path: the stored-layout and decode entries refuse them
    gate_up = torch.zeros(4, 128, 128, dtype=torch.bfloat16, device=device)
    with pytest.raises(RuntimeError):
        ops.moe_experts(d[0], gate_up, d[2].transpose(1, 2).contiguous(), d[3], d[4], 2, act=_native.ACT_RELU)
