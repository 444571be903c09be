"""Seeded sweep of random legal shapes through the three GPU paths, against the fp64 oracle.

The hand-picked cases elsewhere cover the BASELINE shapes and known edge cases; this sweep draws shapes nobody
chose: H and F any multiple of 64 up to 768, 1-40 experts, top-1..8, 1-700 tokens, every layout/activation/bias
combination, invalid slots and skewed routing. Each prefill case runs the packed path (the loaders') and the
stored-layout path (the named C entries) and checks both against the fp64 oracle at the default bar, and each
other at twice it; each decode case checks the gather-GEMV. The shapes come from a fixed seed, so the case list
(and its ids) is the same on every run.
"""

from __future__ import annotations

import random

import pytest

from helpers import TOL_RMS, assert_within_tolerance, half_ulp_bf16, oracle_fp64, rand_case, run_gpu, to_device

pytestmark = pytest.mark.gpu

_COMBOS = [("concat", "silu", False), ("interleaved", "gptoss", True), ("concat", "gptoss", True),
           ("interleaved", "silu", False)]


def _prefill_cases(n=24, seed=20261202):
    r = random.Random(seed)
    out = []
    for i in range(n):
        E = r.randint(1, 40)
        K = r.randint(1, min(E, 8))
        layout, act, bias = _COMBOS[i % len(_COMBOS)]
        out.append((1000 + i, r.randint(1, 700), 64 * r.randint(1, 12), 64 * r.randint(1, 12), E, K, layout, act,
                    bias, r.randint(0, 3) if E > 1 else 0, r.choice([0.0, 0.0, 1.0, 2.0])))
    return out


def _decode_cases(n=16, seed=20261203):
    r = random.Random(seed)
    out = []
    for i in range(n):
        E = r.randint(1, 64)
        K = r.randint(1, min(E, 8))
        T = r.randint(1, min(64, 256 // K))
        act, bias = (("silu", False), ("gptoss", True))[i % 2]
        out.append((2000 + i, T, 64 * r.randint(1, 12), 64 * r.randint(1, 12), E, K, act, bias))
    return out


@pytest.mark.parametrize("case", _prefill_cases(), ids=lambda c: f"T{c[1]}H{c[2]}F{c[3]}E{c[4]}k{c[5]}{c[6]}{c[7]}")
def test_sweep_prefill(device, case):
    from cernels_amd import ops

    seed, T, H, Fi, E, K, layout, act, bias, invalid, skew = case
    c = rand_case(seed, T, H, Fi, E, K, layout=layout, act=act, bias=bias, invalid=invalid, skew=skew,
                  std=0.05 if act == "gptoss" else 0.02)
    print(f"[sweep prefill {case}]", flush=True)
    ref = oracle_fp64(c)
    d = to_device(c, device)
    lay = ops.LAYOUT_CONCAT if layout == "concat" else ops.LAYOUT_INTERLEAVED
    ac = ops.ACT_SILU if act == "silu" else ops.ACT_GPTOSS
    pk = ops.pack_experts(d["W1"], d["W2"], layout=lay, act=ac, gate_up_bias=d["b1"], down_bias=d["b2"])
    packed = ops.moe_experts_packed(d["x"], pk, d["idx"], d["w"], K).cpu()
    stored = run_gpu(c, device, dev_tensors=d).cpu()
    assert_within_tolerance(packed, ref, f"packed {case}")
    assert_within_tolerance(stored, ref, f"stored {case}")
    # the two paths round glu and Y differently; each is within the bar (plus half a bf16 ulp) of the exact value,
    # so they are within twice it of each other
    rms = ref.double().pow(2).mean().sqrt().item()
    gap = ((packed.double() - stored.double()).abs() - 2 * half_ulp_bf16(ref.double())).max().item()
    assert gap <= 2 * TOL_RMS * rms, f"packed vs stored {case}: {gap:.3e} > {2 * TOL_RMS}*RMS({rms:.3e})"


@pytest.mark.parametrize("case", _decode_cases(), ids=lambda c: f"T{c[1]}H{c[2]}F{c[3]}E{c[4]}k{c[5]}{c[6]}")
def test_sweep_decode(device, case):
    seed, T, H, Fi, E, K, act, bias = case
    c = rand_case(seed, T, H, Fi, E, K, layout="concat", act=act, bias=bias, std=0.05 if bias else 0.02)
    print(f"[sweep decode {case}]", flush=True)
    out = run_gpu(c, device, decode=True).cpu()
    assert_within_tolerance(out, oracle_fp64(c), f"decode {case}")
