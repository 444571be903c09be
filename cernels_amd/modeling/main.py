"""Whole-model benchmark, stock vs swapped experts: prefill latency and decode throughput.

Usage: python -m cernels_amd.modeling.main <model> [--checkpoint DIR] [--layers N] ...
       (<model> = north_mini_code | deepseek_ocr_2, an entry of cernels_amd.modeling.swaps.SWAPS)

Same protocol as the reference's src/modeling/main.py:48-95. For every variant, stock first:
  - a correctness gate vs stock: greedy-token prefix match over ``--gate-tokens``, and the max abs
    diff of the last prefill logits (reported, not gated), calibrated by the same two numbers for
    stock under transformers' other experts implementation (``stock_drift_calibration``);
  - prefill latency: torch.utils.benchmark median of ``model(**inputs)``;
  - decode tokens/s: ``decode_tokens / (generate wall - prefill)``, best of ``--runs`` generates.
The model is the real transformers architecture, from a local checkpoint directory or with seeded
random weights (cernels_amd.modeling.models), fed seeded random token ids. The result is written
as JSON (``--out``) and printed.
"""

from __future__ import annotations

import argparse
import json
import platform
import sys
import time
from pathlib import Path

import torch

from cernels_amd.modeling import models as M
from cernels_amd.modeling.swaps import SWAPS

GATE_TOKENS = 64
DECODE_TOKENS = 128


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


@torch.no_grad()
def greedy(model, inputs, n):
    out = model.generate(**inputs, max_new_tokens=n, min_new_tokens=n, do_sample=False)
    return out[0, inputs["input_ids"].size(1):]


@torch.no_grad()
def last_logits(model, inputs):
    return model(**inputs).logits[0, -1].float()


@torch.no_grad()
def time_generate_s(model, inputs, n, runs=3):
    times = []
    for _ in range(runs):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        model.generate(**inputs, max_new_tokens=n, min_new_tokens=n, do_sample=False)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    return min(times)


@torch.no_grad()
def prefill_s(model, inputs, min_run_time):
    from torch.utils.benchmark import Timer

    m = Timer(stmt="model(**inputs)", globals={"model": model, "inputs": inputs}).blocked_autorange(
        min_run_time=min_run_time)
    return m.median


def run(model, inputs, name, variants=None, gate_tokens=GATE_TOKENS, decode_tokens=DECODE_TOKENS, runs=3,
        min_run_time=5.0):
    apply, all_variants = SWAPS[name]
    variants = list(all_variants if variants is None else variants)
    if variants[0] != "stock":
        variants = ["stock"] + [v for v in variants if v != "stock"]
    results = {}
    ref_tokens = ref_logits = None
    for variant in variants:
        t0 = time.time()
        apply(model, variant)
        tokens, logits = greedy(model, inputs, gate_tokens), last_logits(model, inputs)
        if variant == "stock":
            ref_tokens, ref_logits = tokens, logits
        match = int((tokens == ref_tokens).int().cumprod(0).sum())
        p = prefill_s(model, inputs, min_run_time)
        gen = time_generate_s(model, inputs, decode_tokens, runs)
        results[variant] = {
            "prefill_ms": round(p * 1e3, 2),
            "decode_tok_s": round(decode_tokens / (gen - p), 2),
            "generate_s": round(gen, 3),
            "gate_token_match": f"{match}/{gate_tokens}",
            "last_logits_max_diff": round((logits - ref_logits).abs().max().item(), 4),
            "last_logits_std": round(ref_logits.std().item(), 4),
        }
        _log(f"{variant}: {results[variant]} ({time.time() - t0:.0f} s)")
    apply(model, "stock")
    return results


def stock_drift(model, inputs, gate_tokens=GATE_TOKENS):
    """The gate's calibration: stock under transformers' other experts implementation (grouped_mm
    vs eager) against stock as configured. Two correct bf16 implementations drift apart too; on a
    deep model with random weights they can disagree from the first greedy token."""
    cfg = getattr(model.config, "text_config", model.config)
    current = cfg._experts_implementation
    other = "eager" if current != "eager" else "grouped_mm"
    tokens, logits = greedy(model, inputs, gate_tokens), last_logits(model, inputs)
    try:
        model.set_experts_implementation(other)
    except (ValueError, ImportError) as e:  # grouped_mm may not dispatch on this build
        return {"other": other, "error": str(e)}
    try:
        t2, l2 = greedy(model, inputs, gate_tokens), last_logits(model, inputs)
    finally:
        model.set_experts_implementation(current)
    match = int((t2 == tokens).int().cumprod(0).sum())
    return {"other": other, "gate_token_match": f"{match}/{gate_tokens}",
            "last_logits_max_diff": round((l2 - logits).abs().max().item(), 4)}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("model", choices=sorted(SWAPS))
    ap.add_argument("--checkpoint", help="local transformers checkpoint directory (default: seeded random weights)")
    ap.add_argument("--layers", type=int, help="decoder layers (default: the model's)")
    ap.add_argument("--prefill-tokens", type=int, help="prompt length (default: the reference's)")
    ap.add_argument("--decode-tokens", type=int, default=DECODE_TOKENS)
    ap.add_argument("--gate-tokens", type=int, default=GATE_TOKENS)
    ap.add_argument("--runs", type=int, default=3, help="generate runs per variant (best is kept)")
    ap.add_argument("--min-run-time", type=float, default=5.0, help="seconds of prefill timing per variant")
    ap.add_argument("--variants", help="comma list (stock is always first)")
    ap.add_argument("--stock-experts", choices=["default", "eager", "grouped_mm"], default="default",
                    help="transformers experts implementation of the stock variant")
    ap.add_argument("--out", default="gpurun_out/model", help="directory for <model>.json")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        sys.exit("modeling.main needs a GPU")
    from cernels_amd import _native

    _native.lib()  # the swapped variants need the native library: fail now, not mid-run
    spec = M.SPECS[args.model]
    t0 = time.time()
    model = M.build(spec, "cuda", layers=args.layers, checkpoint=args.checkpoint)
    if args.stock_experts != "default":
        model.set_experts_implementation(args.stock_experts)
    cfg = getattr(model.config, "text_config", model.config)
    inputs = M.prompt_ids(spec, args.prefill_tokens, "cuda", vocab=cfg.vocab_size)
    n_params = sum(p.numel() for p in model.parameters())
    _log(f"{args.model}: {n_params / 1e9:.2f} B parameters built in {time.time() - t0:.0f} s; prefill "
         f"{inputs['input_ids'].shape[1]} tokens, decode {args.decode_tokens}; stock experts "
         f"'{cfg._experts_implementation}', attention '{cfg._attn_implementation}'")
    variants = None if not args.variants else [v.strip() for v in args.variants.split(",") if v.strip()]
    results = run(model, inputs, args.model, variants, args.gate_tokens, args.decode_tokens, args.runs,
                  args.min_run_time)
    drift = stock_drift(model, inputs, args.gate_tokens)
    _log(f"stock drift calibration ({cfg._experts_implementation} vs {drift['other']}): {drift}")
    payload = {
        "model": args.model,
        "weights": args.checkpoint or f"seeded N(0, {M.INIT_STD}) random weights, architecture of the published model",
        "layers": cfg.num_hidden_layers,
        "parameters": n_params,
        "prefill_tokens": int(inputs["input_ids"].shape[1]),
        "decode_tokens": args.decode_tokens,
        "stock_experts_implementation": cfg._experts_implementation,
        "stock_drift_calibration": drift,
        "machine": {"gpu": torch.cuda.get_device_name(0), "host": platform.node(), "torch": torch.__version__},
        "variants": results,
    }
    out = Path(args.out)
    out.mkdir(parents=True, exist_ok=True)
    (out / f"{args.model}.json").write_text(json.dumps(payload, indent=1))
    print(json.dumps(payload, indent=1), flush=True)


if __name__ == "__main__":
    main()
