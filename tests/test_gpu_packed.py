"""Packed-weight prefill: the pack kernel's layout, and parity of the packed grouped GEMMs.

The packed layout is this build's own format (MFMA-fragment order), so it is checked against an
independent numpy construction of the same index map. The packed prefill is then held to the
same bar as the prefill on the transformers layouts: |out - fp64| <= 2e-2*RMS + half a bf16 ulp,
the reference's allclose against op_eager, and — at the BASELINE sizes — agreement with the
unpacked path within tolerance (the packed path multiplies fp16 glu by fp16 weights and stores the
per-pair down rows as 24-bit floats; the unpacked path uses bf16 glu and fp32 rows), plus the strict
bar max|out - fp64| <= 2e-2*RMS over the whole output with no allowance.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN_NAMES, load_golden
from helpers import (assert_reference_verify, assert_strict_full, assert_within_tolerance, full_case, oracle_eager,
                     oracle_fp64, rand_case, run_gpu, to_device)

pytestmark = pytest.mark.gpu


def _np_pack(W: np.ndarray, layout: str, which: int, H: int, F: int) -> np.ndarray:
    """Packed order built fragment by fragment: for tile t (8 fragments), k-step ks, fragment c,
    lane l: 8 elements B[16ks + 8(l//32) + j][column of (c, l%32)]. gate_up fragment c holds gate
    columns 16c..16c+15 then the matching up columns; down fragment c holds columns 32c..32c+31."""
    E = W.shape[0]
    if which == 0:  # B[k][n]: n = gate f or up f
        Bk = np.transpose(W, (0, 2, 1)) if layout == "concat" else W  # [E, H, 2F] (concat: gate|up; interleaved: g,u,...)
        if layout == "concat":
            gate, up = Bk[:, :, :F], Bk[:, :, F:]
        else:
            gate, up = Bk[:, :, 0::2], Bk[:, :, 1::2]
        NF, KS = F // 16, H // 16
        col = lambda e, c, j: (gate if j < 16 else up)[e, :, 16 * c + j % 16]  # noqa: E731
    else:
        Bk = np.transpose(W, (0, 2, 1)) if layout == "concat" else W  # [E, F, H]
        NF, KS = H // 32, F // 16
        col = lambda e, c, j: Bk[e, :, 32 * c + j]  # noqa: E731
    out = []
    for e in range(E):
        for t in range((NF + 7) // 8):
            frags = list(range(8 * t, min(8 * t + 8, NF)))
            for ks in range(KS):
                for c in frags:
                    frag = np.empty((64, 8), dtype=W.dtype)
                    for lane in range(64):
                        k0 = 16 * ks + 8 * (lane // 32)
                        frag[lane] = col(e, c, lane % 32)[k0:k0 + 8]
                    out.append(frag.reshape(-1))
    return np.concatenate(out)


@pytest.mark.parametrize("layout", ["concat", "interleaved"])
@pytest.mark.parametrize("which", [0, 2])
def test_pack_layout_bf16(device, layout, which):
    """gate_up (which 0) and the non-gated first projection (which 2, a down-shaped bf16 pack with H and F
    exchanged) keep the source bits: random bit patterns land in the fragment order."""
    from cernels_amd import ops

    H, F, E = 192, 320, 2  # 20 gate_up / 10 up fragments: partial last tiles
    g = torch.Generator().manual_seed(3)
    if which == 0:
        shape = (E, 2 * F, H) if layout == "concat" else (E, H, 2 * F)
    else:  # UP: concat [E, F, H] (rows are outputs), interleaved [E, H, F]
        shape = (E, F, H) if layout == "concat" else (E, H, F)
    W = torch.randint(-30000, 30000, shape, generator=g, dtype=torch.int16)
    Wd = W.view(torch.bfloat16).contiguous().to(device)
    lay = ops.LAYOUT_CONCAT if layout == "concat" else ops.LAYOUT_INTERLEAVED
    got = ops.pack_weights(Wd, lay, which, H, F).view(torch.int16).cpu().numpy()
    want = _np_pack(W.numpy(), layout, 0 if which == 0 else 1, F if which == 2 else H, H if which == 2 else F)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("layout", ["concat", "interleaved"])
def test_pack_layout_down_fp16(device, layout):
    """down: fp16 fragments, each 32-output-column fragment scaled by 2^-s with s = frexp exponent of its
    largest |w| minus 15 (so that largest value lands in [2^14, 2^15)), then a table of s per (expert,
    fragment). Columns of different fragments get magnitudes 2^-20..2^10 so every fragment has its own s,
    and one fragment is all zero (s = 0)."""
    from cernels_amd import ops

    H, F, E = 192, 320, 2
    NF = H // 32
    g = torch.Generator().manual_seed(5)
    shape = (E, H, F) if layout == "concat" else (E, F, H)
    W = torch.randn(shape, generator=g)
    col_scale = torch.exp2(torch.arange(E * NF, dtype=torch.float32).reshape(E, NF) * 5.0 - 20.0)
    col_scale[1, 3] = 0.0
    cs = col_scale.repeat_interleave(32, dim=1)  # [E, H]
    W = W * (cs[:, :, None] if layout == "concat" else cs[:, None, :])
    Wb = W.bfloat16()
    lay = ops.LAYOUT_CONCAT if layout == "concat" else ops.LAYOUT_INTERLEAVED
    got = ops.pack_weights(Wb.contiguous().to(device), lay, 1, H, F).cpu().numpy()
    wf = Wb.float().numpy()
    a = np.abs(wf if layout == "concat" else np.transpose(wf, (0, 2, 1)))  # [E, H, F]
    mx = a.reshape(E, NF, 32 * F).max(axis=2)
    s = np.where(mx > 0, np.frexp(mx)[1] - 15, 0).astype(np.int8)
    sc = np.repeat(np.exp2(-s.astype(np.float64)), 32, axis=1)  # [E, H]
    scaled = wf * (sc[:, :, None] if layout == "concat" else sc[:, None, :])
    want = _np_pack(scaled.astype(np.float16).view(np.int16), layout, 1, H, F)
    nfrag = E * H * F * 2
    np.testing.assert_array_equal(got[:nfrag].view(np.int16), want)
    np.testing.assert_array_equal(got[nfrag:nfrag + E * NF].view(np.int8), s.reshape(-1))


def _run_packed(c, device, d=None):
    from cernels_amd import ops

    d = d or to_device(c, device)
    layout = ops.LAYOUT_CONCAT if c["layout"] == "concat" else ops.LAYOUT_INTERLEAVED
    act = ops.ACT_SILU if c["act"] == "silu" else ops.ACT_GPTOSS
    pk = ops.pack_experts(d["W1"], d["W2"], layout=layout, act=act, gate_up_bias=d["b1"], down_bias=d["b2"])
    return ops.moe_experts_packed(d["x"], pk, d["idx"], d["w"], d["idx"].shape[1])


SMALL = [
    # (seed, T, H, F, E, K, layout, act, bias, invalid, skew)
    (0, 37, 128, 64, 8, 3, "concat", "silu", False, 0, 0.0),
    (1, 300, 256, 192, 16, 4, "concat", "silu", False, 3, 0.0),
    (2, 513, 64, 128, 5, 2, "concat", "silu", False, 0, 3.0),
    (3, 100, 192, 128, 4, 2, "interleaved", "gptoss", True, 0, 0.0),
    (4, 250, 320, 192, 6, 3, "interleaved", "gptoss", True, 2, 0.0),
    (5, 64, 128, 128, 3, 1, "interleaved", "silu", False, 0, 0.0),
    (6, 90, 128, 64, 8, 2, "concat", "gptoss", True, 0, 0.0),
    (7, 1, 128, 64, 16, 8, "concat", "silu", False, 0, 0.0),
    (8, 1200, 256, 128, 64, 6, "concat", "silu", False, 0, 1.2),
    (9, 700, 576, 320, 3, 2, "concat", "silu", False, 0, 0.0),  # 20 and 18 fragments: idle waves in the last tile
    # routes past the one-launch route's LDS limit (the GEMMs' work counters are then zeroed by the scan launch)
    (10, 6000, 64, 64, 1024, 4, "concat", "silu", False, 5, 0.0),
    (11, 8192, 64, 64, 1024, 8, "concat", "silu", False, 0, 1.0),
]


@pytest.mark.parametrize("case", SMALL, ids=lambda c: f"T{c[1]}H{c[2]}F{c[3]}E{c[4]}k{c[5]}{c[6]}")
def test_packed_small(device, case):
    seed, T, H, Fi, E, K, layout, act, bias, invalid, skew = case
    c = rand_case(seed, T, H, Fi, E, K, layout=layout, act=act, bias=bias, invalid=invalid, skew=skew,
                  std=0.05 if act == "gptoss" else 0.02)
    print(f"[packed small {case}]", flush=True)
    out = _run_packed(c, device).cpu()
    assert_within_tolerance(out, oracle_fp64(c), str(case))
    assert_reference_verify(out, oracle_eager(c), str(case))


def test_packed_cost_split_many_rounds(device):
    """2048 tokens x 8 of 16 experts with skewed routing, F = 4096: ~2200 items, so each of the 256
    workgroups runs 8+ rounds and the route writes cost-balanced per-XCD item ranges, over M-tiles of
    many sizes. A sample of 160 tokens is checked against the fp64 oracle and the reference's
    op_eager bar."""
    c = rand_case(31, 2048, 128, 4096, 16, 8, skew=1.5)
    runs = torch.bincount(c["idx"].flatten(), minlength=16)
    assert int((-(-runs // 256)).sum()) * 32 >= 8 * 8 * 32  # >= 8 rounds at fw = 8 on 256 CUs
    print("[packed cost split] T2048 H128 F4096 E16 k8", flush=True)
    out = _run_packed(c, device).cpu()
    rows = torch.randperm(2048, generator=torch.Generator().manual_seed(5))[:160]
    assert_within_tolerance(out[rows], oracle_fp64(c, rows), "cost split")
    assert_reference_verify(out[rows], oracle_eager(c, rows), "cost split")


@pytest.mark.parametrize("T", [3200, 4096], ids=["count_scan_route", "two_launch_route"])
def test_packed_cost_split_other_route_kernels(device, T):
    """The same per-XCD split written by the route's other two kernels: E = 1024 experts with
    T x 8 pairs is past the one-launch route's LDS (count + scan in one launch at 25 route tiles,
    separate launches at 32), and ~4000 small items give every workgroup 8+ rounds."""
    c = rand_case(41, T, 64, 512, 1024, 8, skew=1.0)
    print(f"[packed cost split, route T={T}] H64 F512 E1024 k8", flush=True)
    out = _run_packed(c, device).cpu()
    rows = torch.randperm(T, generator=torch.Generator().manual_seed(6))[:256]
    assert_within_tolerance(out[rows], oracle_fp64(c, rows), f"cost split route T={T}")
    assert_reference_verify(out[rows], oracle_eager(c, rows), f"cost split route T={T}")


@pytest.mark.parametrize("name", GOLDEN_NAMES)
def test_packed_golden(device, name):
    t, meta = load_golden(name)
    c = dict(x=t["x"], idx=t["top_k_index"], w=t["top_k_weights"], W1=t["gate_up_proj"], W2=t["down_proj"],
             b1=t.get("gate_up_proj_bias"), b2=t.get("down_proj_bias"), layout=meta["layout"], act=meta["act"])
    out = _run_packed(c, device).cpu()
    assert_reference_verify(out, t["out"], name)
    assert_within_tolerance(out, oracle_fp64(c), name)


@pytest.mark.parametrize("name", ["deepseek_v2_lite_prefill", "a3b_30b_prefill", "gpt_oss_20b_experts", "qwen3_next_zipf"])
def test_packed_baseline_full_size(device, name):
    from cernels_amd.configs.registry import BASELINE_SHAPES
    from cernels_amd.configs.synth import make_inputs, make_weights

    s = BASELINE_SHAPES[name]
    print(f"[packed full {name}] generating", flush=True)
    inp, wts = make_inputs(s), make_weights(s)
    c = dict(x=inp.x, idx=inp.top_k_index, w=inp.top_k_weights, W1=wts.gate_up_proj, W2=wts.down_proj,
             b1=wts.gate_up_proj_bias, b2=wts.down_proj_bias, layout=s.layout, act=s.act)
    d = to_device(c, device)
    print(f"[packed full {name}] run", flush=True)
    out = _run_packed(c, device, d)
    out2 = _run_packed(c, device, d)
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), "not run-to-run deterministic"
    ref_native = run_gpu(c, device, dev_tensors=d)
    same = torch.equal(out.view(torch.int16), ref_native.view(torch.int16))
    rows = torch.randperm(s.tokens, generator=torch.Generator().manual_seed(0))[:48]
    st = assert_within_tolerance(out.cpu()[rows], oracle_fp64(c, rows), name, strict=True)
    print(f"[packed full {name}] max|err|/RMS = {st['ratio']:.4f}; bit-identical to unpacked path: {same} "
          "(not expected: fp16 glu and 24-bit rows vs bf16 glu and fp32 rows)", flush=True)
    assert_reference_verify(out.cpu()[rows], oracle_eager(c, rows), name)
    assert_within_tolerance(out.cpu(), ref_native.cpu().double(), f"{name} packed vs unpacked")


@pytest.mark.parametrize("name", ["deepseek_v2_lite_prefill", "a3b_30b_prefill", "gpt_oss_20b_experts", "qwen3_next_zipf",
                                  "cohere2_moe_experts", "deepseek_ocr2_moe_experts"])
def test_packed_full_output_strict(device, name):
    """The north-star bar on the WHOLE [T, H] output of each BASELINE prefill workload, and of the reference's
    own prefill configs with their own routings (cohere2: top-k of the logits then sigmoid, no renorm,
    src/configs/registry/cohere2_moe_experts.py:76-78; deepseek: softmax then top-k, no renorm,
    deepseek_ocr2_moe_experts.py:80-83), with no allowance: max|out - exact| <= 2e-2 * RMS(exact), the
    exact value being the float64 restatement of the op on the same bf16 inputs (computed on the GPU in
    float64 by the oracle; checker only). The correctly rounded answer bf16(exact) is measured beside it,
    as the floor any bf16 output has."""
    c, d, ref = full_case(name, device)
    out = _run_packed(c, device, d)
    assert_strict_full(out, ref, f"packed {name}")


def _scaled_rows_case(seed, T, H, Fi, E, K, big_rows, gain, bias=False):
    c = rand_case(seed, T, H, Fi, E, K, std=0.05, bias=bias)
    x = c["x"].float()
    x[big_rows] *= gain
    c["x"] = x.bfloat16()
    return c


@pytest.mark.parametrize("gain,bias", [(300.0, False), (3000.0, False), (3000.0, True)])
def test_glu_beyond_fp16_range_is_rescaled(device, gain, bias):
    """glu is stored in fp16: a segment whose |glu| reaches 2^15 is stored scaled, its row is brought to
    one scale between the GEMMs, and the combine scales that pair's row back (and adds the down bias
    unscaled). Rows of x multiplied by `gain` make silu(g)*u reach ~1e5-1e7 on those rows only; every
    row, scaled or not, must meet the bar on its own scale (the fp64 oracle per row group), and the
    output must be finite."""
    T, H, Fi, E, K = 300, 256, 192, 8, 3
    big = torch.arange(0, T, 37)
    c = _scaled_rows_case(11, T, H, Fi, E, K, big, gain, bias)
    out = _run_packed(c, device).cpu()
    assert torch.isfinite(out.float()).all()
    ref = oracle_fp64(c)
    small = torch.ones(T, dtype=torch.bool)
    small[big] = False
    assert_within_tolerance(out[big], ref[big], f"scaled rows gain {gain}")
    assert_within_tolerance(out[small], ref[small], f"other rows gain {gain}")


@pytest.mark.parametrize("gain", [1e-3, 1e-4])
def test_small_glu_is_rescaled(device, gain):
    """glu is stored in fp16, whose subnormals (below 2^-14) have a fixed 2^-24 spacing: a row of tiny glu
    values would lose most of its precision. Segments whose largest |glu| is below 2^-8 are stored scaled
    up, and the row is brought to one scale as above. Rows of x multiplied by `gain` (glu ~ gain^2:
    3e-7 and 3e-9 here) must each meet the bar on their own scale; so must the rows left alone."""
    T, H, Fi, E, K = 300, 256, 192, 8, 3
    tiny = torch.arange(5, T, 23)
    c = _scaled_rows_case(13, T, H, Fi, E, K, tiny, gain)
    out = _run_packed(c, device).cpu()
    ref = oracle_fp64(c)
    rest = torch.ones(T, dtype=torch.bool)
    rest[tiny] = False
    assert float(ref[tiny].abs().max()) < 1e-4 * float(ref[rest].abs().max())
    assert_within_tolerance(out[tiny], ref[tiny], f"tiny rows gain {gain}", strict=True)
    assert_within_tolerance(out[rest], ref[rest], f"other rows gain {gain}")


def test_small_zero_and_normal_segments_in_one_row(device):
    """Rows whose glu segments differ in scale: for two experts the gate and up weights of intermediate
    columns 0-15 are multiplied by 1e-4 (a tiny segment beside normal ones: the row keeps scale 0 and the
    tiny segment is brought back to it) and those of columns 16-31 are zero (an all-zero segment, exact at
    any scale); rows of x scaled by 1e-3 then have only tiny and zero segments and are scaled up as a
    whole. Every row group meets the bar on its own scale."""
    T, H, Fi, E, K = 256, 128, 128, 4, 2
    c = rand_case(14, T, H, Fi, E, K, std=0.05)
    W1 = c["W1"].float()
    for e in (0, 2):
        for half in (0, Fi):  # gate rows, then the matching up rows
            W1[e, half:half + 16] *= 1e-4
            W1[e, half + 16:half + 32] = 0.0
    c["W1"] = W1.bfloat16()
    tiny = torch.arange(0, T, 9)
    x = c["x"].float()
    x[tiny] *= 1e-3
    c["x"] = x.bfloat16()
    out = _run_packed(c, device).cpu()
    ref = oracle_fp64(c)
    rest = torch.ones(T, dtype=torch.bool)
    rest[tiny] = False
    assert_within_tolerance(out[tiny], ref[tiny], "tiny rows with zero segments", strict=True)
    assert_within_tolerance(out[rest], ref[rest], "rows with a tiny and a zero segment")


def test_glu_beyond_fp16_range_nongated(device):
    """The non-gated first projection (megablocks' w1) with ReLU and rows of x scaled up: its fp16 glu
    segments of 32 columns take the same rescaling path."""
    from cernels_amd import ops
    from oracle import eager as O

    g = torch.Generator().manual_seed(12)
    T, H, F, E, K = 200, 128, 192, 4, 2
    x = torch.randn(T, H, generator=g)
    big = torch.arange(3, T, 29)
    x[big] *= 2000.0
    x = x.bfloat16()
    w1 = (torch.randn(E, H, F, generator=g) * 0.05).bfloat16()
    w2 = (torch.randn(E, F, H, generator=g) * 0.05).bfloat16()
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).int()
    wt = torch.rand(T, K, generator=g)
    d = [t.contiguous().to(device) for t in (x, w1, w2, idx, wt)]
    out = ops.megablocks_moe(*d, K, 2).cpu()
    ref = O.megablocks_fp64(x, idx, wt, w1, w2, 2)
    small = torch.ones(T, dtype=torch.bool)
    small[big] = False
    assert torch.isfinite(out.float()).all()
    assert_within_tolerance(out[big], ref[big], "relu scaled rows")
    assert_within_tolerance(out[small], ref[small], "relu other rows")


def test_small_glu_nongated(device):
    """The non-gated projection (ReLU: many all-zero 32-column segments) with rows of x scaled by 1e-4: the
    tiny rows are scaled up past their zero segments and meet the bar on their own scale."""
    from cernels_amd import ops
    from oracle import eager as O

    g = torch.Generator().manual_seed(15)
    T, H, F, E, K = 200, 128, 192, 4, 2
    x = torch.randn(T, H, generator=g)
    tiny = torch.arange(1, T, 13)
    x[tiny] *= 1e-4
    x = x.bfloat16()
    w1 = (torch.randn(E, H, F, generator=g) * 0.05).bfloat16()
    w2 = (torch.randn(E, F, H, generator=g) * 0.05).bfloat16()
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).int()
    wt = torch.rand(T, K, generator=g)
    d = [t.contiguous().to(device) for t in (x, w1, w2, idx, wt)]
    out = ops.megablocks_moe(*d, K, 2).cpu()
    ref = O.megablocks_fp64(x, idx, wt, w1, w2, 2)
    rest = torch.ones(T, dtype=torch.bool)
    rest[tiny] = False
    assert_within_tolerance(out[tiny], ref[tiny], "relu tiny rows", strict=True)
    assert_within_tolerance(out[rest], ref[rest], "relu other rows")


@pytest.mark.parametrize("layout,act,bias", [("concat", "silu", False), ("interleaved", "gptoss", True)],
                         ids=["silu", "gptoss"])
def test_packed_nan_token_rows(device, layout, act, bias):
    """A token whose hidden state holds a nan gives an all-nan output row, through the glu segments (a nan
    is passed over by the segment maximum), the 24-bit Y rows (a nan stays a nan) and the combine; every
    other token's row is within the bar of the fp64 oracle."""
    c = rand_case(61, 300, 256, 192, 8, 3, layout=layout, act=act, bias=bias, std=0.05 if bias else 0.02)
    bad = torch.tensor([0, 17, 299])
    c["x"][bad, 5] = float("nan")
    print(f"[packed nan rows {layout}]", flush=True)
    out = _run_packed(c, device).cpu()
    assert torch.isnan(out[bad].float()).all()
    keep = torch.tensor([t for t in range(300) if t not in bad.tolist()])
    assert not torch.isnan(out[keep].float()).any()
    assert_within_tolerance(out[keep], oracle_fp64(c, keep), f"nan rows {layout}")
