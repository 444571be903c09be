"""Pins the CPU oracle (oracle/) before anything is checked against it. CPU only.

* experts_eager  == transformers' eager experts forward, bit for bit, on the golden fixtures.
* route_reference == the golden torch.where visiting order; == oracle/route.c (C restatement).
* experts_fp64   == an independent per-(token, slot) brute force; closed-form special cases.
* the harness routers (cernels_amd.configs.synth.route) == transformers' routers on the fixtures.
"""

from __future__ import annotations

import ctypes
import subprocess

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import GOLDEN_NAMES, ROOT, load_golden
from oracle import eager as O

ORACLE_SO = ROOT / "oracle" / "_build" / "liboracle_route.so"


def _layout_args(t, meta):
    return dict(
        gate_up_bias=t.get("gate_up_proj_bias"),
        down_bias=t.get("down_proj_bias"),
        layout=meta["layout"],
        act=meta["act"],
    )


@pytest.mark.parametrize("name", GOLDEN_NAMES)
def test_eager_restatement_matches_transformers_bitwise(name):
    t, meta = load_golden(name)
    out = O.experts_eager(t["x"], t["top_k_index"], t["top_k_weights"], t["gate_up_proj"], t["down_proj"],
                          **_layout_args(t, meta))
    assert out.dtype == torch.bfloat16
    assert torch.equal(out.view(torch.int16), t["out"].view(torch.int16)), f"{name}: eager restatement drifted"


@pytest.mark.parametrize("name", GOLDEN_NAMES)
def test_route_reference_matches_torch_where_order(name):
    t, meta = load_golden(name)
    r = O.route_reference(t["top_k_index"].numpy(), meta["E"])
    np.testing.assert_array_equal(r["sorted_pairs"], t["where_pairs"].numpy())
    counts = np.bincount(t["top_k_index"].numpy().ravel(), minlength=meta["E"])
    np.testing.assert_array_equal(np.diff(r["offsets"]), counts)


@pytest.mark.parametrize("name", GOLDEN_NAMES)
def test_fp64_close_to_transformers(name):
    """The exact value sits within op_eager's own bf16 noise of transformers' output."""
    t, meta = load_golden(name)
    ref = O.experts_fp64(t["x"], t["top_k_index"], t["top_k_weights"], t["gate_up_proj"], t["down_proj"],
                         **_layout_args(t, meta))
    st = O.error_stats(t["out"], ref)
    assert st["ratio"] < 0.1, st


@pytest.mark.parametrize("family,router", [("cohere2_t16", "topk_sigmoid"), ("cohere2_t1", "topk_sigmoid"),
                                           ("qwen3_t10", "softmax_topk_renorm"), ("gpt_oss_t9", "topk_softmax")])
def test_harness_router_matches_transformers(family, router):
    from cernels_amd.configs.synth import route

    t, meta = load_golden(family)
    idx, w = route(t["logits"].float(), meta["K"], router)
    assert torch.equal(idx, t["top_k_index"])
    assert torch.equal(w.view(torch.int16), t["top_k_weights"].view(torch.int16))


def test_deepseek_router_selects_same_experts():
    """DeepseekOcr2 greedy uses topk(sorted=False): same set and weights per token, slot order may differ."""
    from cernels_amd.configs.synth import route

    t, meta = load_golden("deepseek_t12")
    idx, w = route(t["logits"].float(), meta["K"], "softmax_topk")
    for r in range(idx.shape[0]):
        a = sorted(zip(idx[r].tolist(), w[r].float().tolist()))
        b = sorted(zip(t["top_k_index"][r].tolist(), t["top_k_weights"][r].float().tolist()))
        assert a == b


# ---- C restatement of routing -----------------------------------------------------------------

@pytest.fixture(scope="module")
def c_oracle():
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    lib = ctypes.CDLL(str(ORACLE_SO))
    lib.oracle_route.restype = ctypes.c_int
    return lib


def c_route(lib, idx: np.ndarray, E: int, tile_m: int):
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    T, K = idx.shape
    P = T * K
    cap = (P + tile_m - 1) // tile_m + min(E, P) + 1
    offsets = np.zeros(E + 1, np.int32)
    pairs = np.full(max(P, 1), -1, np.int32)
    toff = np.zeros(E + 1, np.int32)
    texp = np.full(cap, -1, np.int32)
    meta = np.zeros(2, np.int32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    rc = lib.oracle_route(p(idx), T, K, E, tile_m, p(offsets), p(pairs), p(toff), p(texp), p(meta))
    assert rc == 0
    nv = int(meta[1])
    return dict(offsets=offsets, sorted_pairs=pairs[:nv], tile_offsets=toff, tile_expert=texp[: meta[0]],
                num_tiles=int(meta[0]), num_valid=nv)


def _compare_route(a, b):
    for k in ("offsets", "sorted_pairs", "tile_offsets", "tile_expert"):
        np.testing.assert_array_equal(a[k], b[k], err_msg=k)
    assert a["num_tiles"] == b["num_tiles"] and a["num_valid"] == b["num_valid"]


@pytest.mark.parametrize("seed", range(6))
def test_c_route_matches_closed_form(c_oracle, seed):
    rng = np.random.default_rng(seed)
    T = int(rng.integers(0, 300))
    K = int(rng.integers(1, 11))
    E = int(rng.integers(1, 600))
    idx = rng.integers(-2, E + 2, size=(T, K))  # includes out-of-range ids
    for tile_m in (1, 64, 128):
        _compare_route(c_route(c_oracle, idx, E, tile_m), O.route_reference(idx, E, tile_m))


@pytest.mark.parametrize("name", GOLDEN_NAMES)
def test_c_route_matches_golden(c_oracle, name):
    t, meta = load_golden(name)
    r = c_route(c_oracle, t["top_k_index"].numpy(), meta["E"], 128)
    np.testing.assert_array_equal(r["sorted_pairs"], t["where_pairs"].numpy())


def test_route_tiny_brute_force():
    """Tiny case written out by hand: 3 tokens, top-2, 3 experts."""
    idx = np.array([[2, 0], [0, 1], [2, 1]])
    r = O.route_reference(idx, 3, tile_m=1)
    # expert 0: (k=0,t=1)->p=2, (k=1,t=0)->p=1 ; expert 1: (k=1,t=1)->3, (k=1,t=2)->5 ;
    # expert 2: (k=0,t=0)->0, (k=0,t=2)->4
    np.testing.assert_array_equal(r["sorted_pairs"], [2, 1, 3, 5, 0, 4])
    np.testing.assert_array_equal(r["offsets"], [0, 2, 4, 6])
    np.testing.assert_array_equal(r["tile_expert"], [0, 0, 1, 1, 2, 2])


# ---- fp64 restatement ---------------------------------------------------------------------------

def _rand_case(seed, T, H, Fi, E, K, layout="concat", act="silu", bias=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).bfloat16()
    if layout == "concat":
        W1 = (torch.randn(E, 2 * Fi, H, generator=g) * 0.05).bfloat16()
        W2 = (torch.randn(E, H, Fi, generator=g) * 0.05).bfloat16()
    else:
        W1 = (torch.randn(E, H, 2 * Fi, generator=g) * 0.05).bfloat16()
        W2 = (torch.randn(E, Fi, H, generator=g) * 0.05).bfloat16()
    b1 = (torch.randn(E, 2 * Fi, generator=g) * 0.05).bfloat16() if bias else None
    b2 = (torch.randn(E, H, generator=g) * 0.05).bfloat16() if bias else None
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    w = torch.rand(T, K, generator=g).bfloat16()
    return x, idx, w, W1, W2, b1, b2


def _brute_fp64(x, idx, w, W1, W2, b1, b2, layout, act):
    """Independent per-(t, k) loop in float64 (no grouping, no index_add)."""
    T, K = idx.shape
    out = np.zeros((T, x.shape[1]))
    X = x.double().numpy()
    for t in range(T):
        for k in range(K):
            e = int(idx[t, k])
            A = W1[e].double().numpy()
            gu = A @ X[t] if layout == "concat" else X[t] @ A
            if b1 is not None:
                gu = gu + b1[e].double().numpy()
            Fi = gu.shape[0] // 2
            g, u = (gu[:Fi], gu[Fi:]) if layout == "concat" else (gu[0::2], gu[1::2])
            if act == "silu":
                h = g / (1 + np.exp(-g)) * u
            else:
                g = np.minimum(g, 7.0)
                u = np.clip(u, -7.0, 7.0)
                h = (u + 1) * g / (1 + np.exp(-1.702 * g))
            B = W2[e].double().numpy()
            y = B @ h if layout == "concat" else h @ B
            if b2 is not None:
                y = y + b2[e].double().numpy()
            out[t] += float(w[t, k]) * y
    return out


@pytest.mark.parametrize("layout,act,bias", [("concat", "silu", False), ("interleaved", "gptoss", True),
                                             ("concat", "gptoss", True), ("interleaved", "silu", False)])
def test_fp64_matches_brute_force(layout, act, bias):
    x, idx, w, W1, W2, b1, b2 = _rand_case(3, T=7, H=24, Fi=16, E=5, K=3, layout=layout, act=act, bias=bias)
    if act == "gptoss":
        x = x * 8  # drive some pre-activations past the +-7 clamps
    ref = O.experts_fp64(x, idx, w, W1, W2, b1, b2, layout=layout, act=act).numpy()
    np.testing.assert_allclose(ref, _brute_fp64(x, idx, w, W1, W2, b1, b2, layout, act), rtol=1e-12, atol=1e-12)


def test_fp64_dense_mlp_special_case():
    """E=1, k=1, w=1 is the textbook gated MLP: down(silu(gate x) * up x)."""
    x, idx, w, W1, W2, _, _ = _rand_case(4, T=5, H=16, Fi=8, E=1, K=1)
    w = torch.ones_like(w)
    ref = O.experts_fp64(x, idx, w, W1, W2)
    gate = x.double() @ W1[0, :8].double().T
    up = x.double() @ W1[0, 8:].double().T
    dense = (F.silu(gate) * up) @ W2[0].double().T
    torch.testing.assert_close(ref, dense, rtol=1e-13, atol=1e-13)


def test_fp64_zero_weights_and_zero_input():
    x, idx, w, W1, W2, b1, b2 = _rand_case(5, T=6, H=16, Fi=8, E=4, K=2, bias=True)
    assert O.experts_fp64(x, idx, torch.zeros_like(w), W1, W2, b1, b2).abs().max() == 0  # bias is scaled by w too
    assert O.experts_fp64(torch.zeros_like(x), idx, w, W1, W2).abs().max() == 0  # silu(0) = 0


def test_fp64_gptoss_clamp_limits():
    """Gate pre-activations far above 7 behave exactly as gate = 7; up below -7 as up = -7."""
    H, Fi = 8, 4
    x = torch.ones(1, H).bfloat16()
    W1 = torch.zeros(1, H, 2 * Fi).bfloat16()
    W1[0, :, 0::2] = 4.0  # gate = 32
    W1[0, :, 1::2] = -4.0  # up = -32
    W2 = torch.eye(Fi, H).unsqueeze(0).bfloat16()
    idx = torch.zeros(1, 1, dtype=torch.int64)
    w = torch.ones(1, 1).bfloat16()
    out = O.experts_fp64(x, idx, w, W1, W2, layout="interleaved", act="gptoss")
    expect = (-7.0 + 1.0) * 7.0 / (1.0 + np.exp(-1.702 * 7.0))
    np.testing.assert_allclose(out[0, :Fi].numpy(), expect, rtol=1e-13)
    # up = -1 exactly zeroes the output whatever the gate
    W1[0, :, 1::2] = -0.125  # up = -1
    out = O.experts_fp64(x, idx, w, W1, W2, layout="interleaved", act="gptoss")
    assert out.abs().max() == 0


def test_fp64_relabel_invariance_and_linearity():
    x, idx, w, W1, W2, _, _ = _rand_case(6, T=9, H=16, Fi=8, E=6, K=3)
    ref = O.experts_fp64(x, idx, w, W1, W2)
    perm = torch.randperm(6, generator=torch.Generator().manual_seed(0))
    inv = torch.argsort(perm)
    relab = O.experts_fp64(x, inv[idx], w, W1[perm], W2[perm])
    torch.testing.assert_close(ref, relab, rtol=1e-12, atol=1e-12)
    doubled = O.experts_fp64(x, idx, (w.float() * 2).bfloat16(), W1, W2)
    torch.testing.assert_close(doubled, 2 * ref, rtol=1e-13, atol=1e-13)


def test_eager_skips_out_of_range_ids():
    x, idx, w, W1, W2, _, _ = _rand_case(7, T=6, H=16, Fi=8, E=4, K=2)
    bad = idx.clone()
    bad[0, 1] = 4
    bad[3, 0] = -1
    got = O.experts_eager(x, bad, w, W1, W2)
    w2 = w.clone()
    w2[0, 1] = 0
    w2[3, 0] = 0
    fixed = idx.clone()
    fixed[0, 1] = 0
    fixed[3, 0] = 0
    ref64 = O.experts_fp64(x, fixed, w2, W1, W2)
    assert O.error_stats(got, ref64)["ratio"] < 0.05
    torch.testing.assert_close(O.experts_fp64(x, bad, w, W1, W2), ref64, rtol=1e-14, atol=1e-14)


# ---- router restatement -------------------------------------------------------------------------

def _identity_router_inputs(T, E, seed, ties=False):
    g = torch.Generator().manual_seed(seed)
    if ties:
        x = (torch.randint(-4, 5, (T, E), generator=g).float() * 0.25).bfloat16()
    else:  # distinct values per row: a random permutation of an evenly spaced set
        base = torch.linspace(-3.0, 3.0, E)
        x = torch.stack([base[torch.randperm(E, generator=g)] for _ in range(T)]).bfloat16()
        assert all(len(set(r.tolist())) == E for r in x.float())
    return x


@pytest.mark.parametrize("E,K", [(8, 2), (32, 4), (64, 10), (128, 8)])
def test_router_select_matches_module_routers(E, K):
    """With W = I (bf16 identity) the module routers' logits equal x exactly, so their own torch
    code (topk / softmax / renorm) pins router_select on tie-free logits."""
    from cernels_amd.configs.modules import GptOssRouter, Qwen3NextRouter

    x = _identity_router_inputs(50, E, seed=E + K)
    eye = torch.eye(E).bfloat16()
    go = GptOssRouter(E, E, K)
    q3 = Qwen3NextRouter(E, E, K, norm_topk_prob=True)
    with torch.no_grad():
        go.weight.copy_(eye)
        q3.weight.copy_(eye)
    go, q3 = go.bfloat16(), q3.bfloat16()
    with torch.no_grad():
        lg, sg, ig = go(x)
        lq, sq, iq = q3(x)
    assert torch.equal(lg, x) and torch.equal(lq, x)
    idx, w = O.router_select(x, K, O.ROUTER_TOPK_SOFTMAX)
    assert torch.equal(idx, ig) and torch.equal(w, sg)
    idx, w = O.router_select(x, K, O.ROUTER_SOFTMAX_TOPK, renorm=True)
    assert torch.equal(idx, iq) and torch.equal(w, sq)


def test_router_select_closed_forms_and_ties():
    x = _identity_router_inputs(20, 16, seed=3)
    p = torch.softmax(x.float(), dim=-1)
    # k = E: every expert, in descending order; weights are the softmax itself
    for mode in (O.ROUTER_SOFTMAX_TOPK, O.ROUTER_TOPK_SOFTMAX):
        idx, w = O.router_select(x, 16, mode, renorm=False)
        assert torch.equal(torch.gather(p, 1, idx).bfloat16(), w)
        assert torch.equal(idx.sort(dim=1).values, torch.arange(16).expand(20, 16))
    # k = 1 renormalised: the argmax with weight exactly 1
    idx, w = O.router_select(x, 1, O.ROUTER_SOFTMAX_TOPK, renorm=True)
    assert torch.equal(idx[:, 0], x.float().argmax(dim=1)) and bool((w == 1).all())
    # ties go to the lower expert id
    t = torch.tensor([[1.0, 3.0, 3.0, 2.0, 3.0]]).bfloat16()
    idx, _ = O.router_select(t, 2, O.ROUTER_TOPK_SOFTMAX)
    assert idx.tolist() == [[1, 2]]
    idx, _ = O.router_select(t, 4, O.ROUTER_SOFTMAX_TOPK)
    assert idx.tolist() == [[1, 2, 4, 3]]


def test_router_select_orders_by_logit_where_fp32_probs_tie():
    """Two distinct bf16 logits near zero whose fp32 softmax probabilities round equal: the expert
    with the larger logit comes first (the exact probabilities differ), not the lower id."""
    a, b = 2.0 ** -20, 2.0 ** -20 + 2.0 ** -27  # adjacent bf16 values
    t = torch.tensor([[0.0, a, b, -1.0]]).bfloat16()
    lo, hi = t[0, 1].item(), t[0, 2].item()
    assert lo == a and hi == b and hi > lo
    p = torch.softmax(t.float(), dim=-1)
    assert p[0, 1] == p[0, 2]  # the fp32 probabilities tie
    idx, w = O.router_select(t, 3, O.ROUTER_SOFTMAX_TOPK, renorm=False)
    assert idx.tolist() == [[2, 1, 0]]  # the larger logit (id 2) before the lower id with the same fp32 probability
    assert torch.equal(w, torch.gather(p, 1, idx).bfloat16())


def test_router_logits_identity():
    x = _identity_router_inputs(7, 24, seed=9, ties=True)
    assert torch.equal(O.router_logits(x, torch.eye(24).bfloat16()), x)
    b = torch.full((24,), 0.5).bfloat16()
    assert torch.equal(O.router_logits(x, torch.eye(24).bfloat16(), b), (x.double() + 0.5).bfloat16())


@pytest.mark.parametrize("Fs,F", [(96, 32), (64, 64), (80, 64)])
def test_shared_expert_fp64_is_the_module_and_an_extra_expert(Fs, F):
    """shared_expert_fp64 equals the stand-in modules' own forward (MLP in float64, gate in bf16),
    and equals the same MLP split by ops.split_shared_expert into S experts of width F (zero-padded),
    routed for every token with weight sigmoid(gate): the identity the fused qwen3 block relies on."""
    from torch import nn

    from cernels_amd import ops
    from cernels_amd.configs.modules import DenseMlp

    H, T = 64, 20
    g = torch.Generator().manual_seed(Fs + F)
    mlp, sg = DenseMlp(H, Fs), nn.Linear(H, 1, bias=False)
    with torch.no_grad():
        for m in (mlp, sg):
            for p in m.parameters():
                p.copy_((torch.randn(p.shape, generator=g) * 0.1).bfloat16().float())
    x = torch.randn(T, H, generator=g).bfloat16()
    gw, uw, dw, sw = (m.weight.data.bfloat16() for m in (mlp.gate_proj, mlp.up_proj, mlp.down_proj, sg))
    ref = O.shared_expert_fp64(x, gw, uw, dw, sw)
    with torch.no_grad():
        s = torch.sigmoid(sg.bfloat16()(x)).double()
        m = mlp.double()(x.double())
    assert torch.allclose(ref, s * m, rtol=1e-12, atol=1e-14)
    gu, dn = ops.split_shared_expert(gw, uw, dw, F)
    S = -(-Fs // F)
    assert tuple(gu.shape) == (S, 2 * F, H) and tuple(dn.shape) == (S, H, F)
    idx = torch.arange(S).expand(T, S)
    ref2 = O.experts_fp64(x, idx, s.float().expand(T, S), gu, dn)
    assert torch.allclose(ref, ref2, rtol=1e-10, atol=1e-13)
    # a mistake in the split (a dropped block, a transposed down) moves the result
    ref3 = O.experts_fp64(x, idx[:, :1], s.float().expand(T, S)[:, :1], gu, dn)
    assert S == 1 or not torch.allclose(ref, ref3, rtol=1e-6, atol=1e-8)


def _megablocks_case(T=12, H=16, F=24, E=5, K=2, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).bfloat16()
    w1 = (torch.randn(E, H, F, generator=g) * 0.2).bfloat16()
    w2 = (torch.randn(E, F, H, generator=g) * 0.2).bfloat16()
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).int()
    wt = torch.rand(T, K, generator=g)
    return x, w1, w2, idx, wt


def test_megablocks_fp64_brute_force_and_closed_forms():
    """Per-(token, slot) brute force with the activations written out (GELU's tanh form from its
    formula, not torch's), ids outside [0, E) skipped, linearity in the routing weights."""
    import math

    x, w1, w2, idx, wt = _megablocks_case()
    idx[0, 1] = -1
    idx[3, 0] = 5  # == E: skipped
    acts = {0: lambda h: 0.5 * h * (1 + torch.tanh(math.sqrt(2 / math.pi) * (h + 0.044715 * h ** 3))),
            1: lambda h: h / (1 + torch.exp(-h)), 2: lambda h: torch.clamp(h, min=0)}
    for a, fn in acts.items():
        ref = O.megablocks_fp64(x, idx, wt, w1, w2, a)
        bf = torch.zeros(ref.shape, dtype=torch.float64)
        for t in range(x.shape[0]):
            for k in range(idx.shape[1]):
                e = int(idx[t, k])
                if 0 <= e < w1.shape[0]:
                    h = x[t].double() @ w1[e].double()
                    bf[t] += float(wt[t, k]) * (fn(h) @ w2[e].double())
        assert torch.allclose(ref, bf, rtol=1e-12, atol=1e-12), a
        assert torch.allclose(O.megablocks_fp64(x, idx, 2 * wt, w1, w2, a), 2 * ref, rtol=1e-12, atol=1e-12)


def test_megablocks_silu_is_a_gated_expert_with_unit_up():
    """silu(x w1) w2 equals the gated experts' silu(gate) * up with gate = w1ᵀ, up weights 0 and up
    bias 1: ties megablocks_fp64 to experts_fp64, which the golden fixtures pin."""
    x, w1, w2, idx, wt = _megablocks_case(seed=3)
    E, H, F = w1.shape
    gate_up = torch.cat([w1.transpose(1, 2), torch.zeros(E, F, H, dtype=w1.dtype)], dim=1)  # [E, 2F, H]
    bias = torch.cat([torch.zeros(E, F), torch.ones(E, F)], dim=1)
    ref = O.experts_fp64(x, idx, wt, gate_up, w2.transpose(1, 2), gate_up_bias=bias)
    assert torch.allclose(O.megablocks_fp64(x, idx, wt, w1, w2, 1), ref, rtol=1e-12, atol=1e-12)
    # the other activations differ from silu on the same inputs (a swapped act id would show)
    assert not torch.allclose(O.megablocks_fp64(x, idx, wt, w1, w2, 0), ref, rtol=1e-6, atol=1e-8)
