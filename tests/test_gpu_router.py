"""Fused router (cernels_moe_router) against the CPU oracle.

Two steps, so that the one place where rounding order can differ is checked on its own:
  1. logits: each bf16 logit is within one bf16 ulp of the float64 value of x Wᵀ + b rounded once,
     plus the first-order bound on fp32 summation of H products, H·2⁻²⁴·Σ|x_i w_i| (the kernel
     accumulates in fp32 on MFMA; where terms cancel to a logit near zero that bound dominates,
     and torch's own bf16 matmul differs from the float64 value there just the same);
  2. selection: recomputed on the CPU from the kernel's own logits with oracle.router_select, the
     indices must be identical (ties to the lower id) and each weight within one bf16 ulp (the
     kernel's exp and reduction order differ from torch's).
The loaders' end-to-end outputs are checked in test_gpu_loaders.py.
"""

from __future__ import annotations

import pytest
import torch

from oracle import eager as O

pytestmark = pytest.mark.gpu


def _case(seed, T, H, E, bias, std=0.05):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).bfloat16()
    w = (torch.randn(E, H, generator=g) * std).bfloat16()
    b = (torch.randn(E, generator=g) * 0.1).bfloat16() if bias else None
    return x, w, b


def _ulp(v: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |v| (2^(exponent-7)), with a floor for values near zero."""
    a = v.float().abs().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


CASES = [
    # (seed, T, H, E, K, mode, renorm, bias)
    (0, 1, 2048, 128, 8, O.ROUTER_SOFTMAX_TOPK, True, False),
    (1, 37, 192, 8, 2, O.ROUTER_SOFTMAX_TOPK, True, False),
    (2, 300, 2048, 512, 10, O.ROUTER_SOFTMAX_TOPK, True, False),  # qwen3-next shape
    (3, 100, 256, 64, 6, O.ROUTER_SOFTMAX_TOPK, False, False),
    (4, 4096, 2880, 32, 4, O.ROUTER_TOPK_SOFTMAX, True, True),  # gpt-oss-20b shape
    (5, 33, 64, 4, 2, O.ROUTER_TOPK_SOFTMAX, True, True),
    (6, 70, 512, 1000, 16, O.ROUTER_SOFTMAX_TOPK, True, False),  # E not a multiple of 32
    (7, 5, 128, 32, 32, O.ROUTER_TOPK_SOFTMAX, True, True),  # k = E = the largest k
    (8, 64, 2048, 512, 1, O.ROUTER_SOFTMAX_TOPK, True, False),  # k = 1
    (9, 129, 80, 48, 5, O.ROUTER_TOPK_SOFTMAX, True, True),  # H % 64 != 0, 32 < E <= 64 (fused)
    (10, 257, 208, 96, 8, O.ROUTER_SOFTMAX_TOPK, False, True),  # H % 64 != 0, E > 64 (GEMM + select)
    (11, 1, 2880, 32, 4, O.ROUTER_TOPK_SOFTMAX, True, True),  # gpt-oss decode
    (12, 8, 2048, 512, 10, O.ROUTER_SOFTMAX_TOPK, True, False),  # qwen3-next decode
    (13, 200, 128, 65, 3, O.ROUTER_TOPK_SOFTMAX, True, False),  # E = 65: smallest unfused
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"T{c[1]}H{c[2]}E{c[3]}k{c[4]}m{c[5]}")
def test_router_matches_oracle(device, case):
    from cernels_amd import ops

    seed, T, H, E, K, mode, renorm, bias = case
    x, w, b = _case(seed, T, H, E, bias)
    print(f"[router {case}]", flush=True)
    idx, wts, logits = ops.moe_router(x.to(device), w.to(device), None if b is None else b.to(device), K, mode,
                                      renorm=renorm, want_logits=True)
    idx, wts, logits = idx.cpu(), wts.cpu(), logits.cpu()
    ref_logits = O.router_logits(x, w, b)
    dl = (logits.float() - ref_logits.float()).abs().double()
    mag = x.double().abs() @ w.double().abs().T
    tol = _ulp(ref_logits).double() + H * 2.0 ** -24 * mag
    assert bool((dl <= tol).all()), f"logits off by more than the bound: {(dl - tol).max()}"
    ridx, rw = O.router_select(logits, K, mode, renorm=renorm)
    assert torch.equal(idx.long(), ridx), "selection differs from the oracle on the kernel's own logits"
    dw = (wts - rw.float()).abs()
    assert bool((dw <= _ulp(rw)).all()), f"weights off by more than one bf16 ulp: {dw.max()}"
    assert torch.equal(wts, wts.bfloat16().float()), "weights must be bf16 values"


def test_router_ties_go_to_lower_id(device):
    from cernels_amd import ops

    # x with repeated columns and W = I: many exactly equal logits per token
    T, E = 64, 32
    g = torch.Generator().manual_seed(11)
    x = (torch.randint(-3, 4, (T, E), generator=g).float() * 0.5).bfloat16()
    w = torch.eye(E).bfloat16()
    for mode in (O.ROUTER_SOFTMAX_TOPK, O.ROUTER_TOPK_SOFTMAX):
        idx, wts = ops.moe_router(x.to(device), w.to(device), None, 6, mode)
        ridx, rw = O.router_select(x, 6, mode)
        assert torch.equal(idx.cpu().long(), ridx)
        assert bool(((wts.cpu() - rw.float()).abs() <= _ulp(rw)).all())


def test_router_feeds_the_experts_op(device):
    """Router output goes straight into the prefill op; equal to routing done by the oracle."""
    from cernels_amd import ops
    from helpers import assert_within_tolerance

    T, H, Fi, E, K = 200, 256, 128, 16, 4
    x, w, _ = _case(21, T, H, E, False)
    g = torch.Generator().manual_seed(22)
    W1 = (torch.randn(E, 2 * Fi, H, generator=g) * 0.02).bfloat16()
    W2 = (torch.randn(E, H, Fi, generator=g) * 0.02).bfloat16()
    idx, wts, logits = ops.moe_router(x.to(device), w.to(device), None, K, ops.ROUTER_SOFTMAX_TOPK, want_logits=True)
    pk = ops.pack_experts(W1.to(device), W2.to(device), layout=ops.LAYOUT_CONCAT, act=ops.ACT_SILU)
    out = ops.moe_experts_packed(x.to(device), pk, idx, wts, K).cpu()
    ridx, rw = O.router_select(logits.cpu(), K, O.ROUTER_SOFTMAX_TOPK)
    ref = O.experts_fp64(x, ridx, rw, W1, W2)
    assert_within_tolerance(out, ref, "router -> experts")


def test_router_rejects_bad_shapes(device):
    from cernels_amd import ops

    x, w, _ = _case(0, 4, 64, 8, False)
    with pytest.raises(RuntimeError):
        ops.moe_router(x.to(device), w.to(device), None, 9, ops.ROUTER_SOFTMAX_TOPK)  # k > E
    x3, w3, _ = _case(0, 4, 64, 64, False)
    with pytest.raises(RuntimeError):
        ops.moe_router(x3.to(device), w3.to(device), None, 33, ops.ROUTER_SOFTMAX_TOPK)  # k > 32
    x2, w2, _ = _case(0, 4, 72, 8, False)
    with pytest.raises(RuntimeError):
        ops.moe_router(x2.to(device), w2.to(device), None, 2, ops.ROUTER_SOFTMAX_TOPK)  # H % 16 != 0


@pytest.mark.parametrize("E,S,mode", [(16, 1, O.ROUTER_SOFTMAX_TOPK), (31, 1, O.ROUTER_SOFTMAX_TOPK),
                                      (40, 2, O.ROUTER_TOPK_SOFTMAX), (63, 3, O.ROUTER_SOFTMAX_TOPK),
                                      (512, 1, O.ROUTER_SOFTMAX_TOPK)])
def test_router_shared_slots(device, E, S, mode):
    """The weight's last row is the shared-expert gate: slots K..K+S-1 get ids E..E+S-1 and weight
    bf16(sigmoid(gate logit)); the routed slots are chosen among the first E logits only."""
    from cernels_amd import ops

    T, H, K = 150, 256, 4
    bias = mode == O.ROUTER_TOPK_SOFTMAX
    x, w, b = _case(31 + E, T, H, E + 1, bias)
    print(f"[router shared E={E} S={S} mode={mode}]", flush=True)
    idx, wts, logits = ops.moe_router(x.to(device), w.to(device), None if b is None else b.to(device), K, mode,
                                      want_logits=True, shared_slots=S)
    idx, wts, logits = idx.cpu(), wts.cpu(), logits.cpu()
    assert tuple(idx.shape) == (T, K + S) and tuple(logits.shape) == (T, E + 1)
    ref_logits = O.router_logits(x, w, b)
    dl = (logits.float() - ref_logits.float()).abs().double()
    tol = _ulp(ref_logits).double() + H * 2.0 ** -24 * (x.double().abs() @ w.double().abs().T)
    assert bool((dl <= tol).all())
    ridx, rw = O.router_select(logits[:, :E], K, mode)
    assert torch.equal(idx[:, :K].long(), ridx)
    assert bool(((wts[:, :K] - rw.float()).abs() <= _ulp(rw)).all())
    assert torch.equal(idx[:, K:], (E + torch.arange(S, dtype=torch.int32)).expand(T, S))
    sg = torch.sigmoid(logits[:, E:].float()).bfloat16()
    assert bool(((wts[:, K:] - sg.float()).abs() <= _ulp(sg)).all())
