"""Whole-model benchmark, stock vs swapped experts: prefill latency and decode throughput.

Usage: python -m cernels_amd.modeling.main <model> [--checkpoint DIR] [--layers N] ...
       (<model> = north_mini_code | deepseek_ocr_2, an entry of cernels_amd.modeling.swaps.SWAPS)

The protocol is the reference's (src/modeling/main.py:1-8, :51-76): each variant of the model's
swap entry, stock first, is
  - gated against stock by the length of the common prefix of their greedy continuations
    (``--gate-tokens``) and by the largest difference of their last-position prefill logits
    (reported, not gated);
  - timed for prefill (median of repeated forwards of the prompt);
  - timed for decode (tokens per second of a fixed-length greedy generate, prefill subtracted).
Two correct bf16 implementations drift apart on a deep model too, so the same two gate numbers are
also measured between stock and stock under transformers' other experts implementation
(``stock_drift_calibration``). The model is the real transformers architecture, from a local
checkpoint directory or with seeded random weights (cernels_amd.modeling.models), fed seeded random
token ids. The result is written as JSON to ``<out>/<host>/model/<model>.json`` (``--out``, default
``analysis``; ``python -m cernels_amd.modeling.view`` tabulates the saved results) and printed.
"""

from __future__ import annotations

import argparse
import json
import platform
import statistics
import sys
import time
from dataclasses import dataclass
from pathlib import Path

import torch

from cernels_amd.modeling import models as M
from cernels_amd.modeling.swaps import SWAPS


@dataclass
class Options:
    gate_tokens: int = 64     # greedy continuation compared against stock
    decode_tokens: int = 128  # tokens generated per decode timing run
    decode_runs: int = 3      # decode timing runs; the fastest is kept
    prefill_seconds: float = 5.0  # time budget of the prefill repeats


@dataclass
class Trace:
    """What a model variant answers on the fixed prompt: its greedy continuation and the fp32 logits
    of the prompt's last position."""

    tokens: torch.Tensor
    logits: torch.Tensor

    def against(self, ref: "Trace") -> dict:
        n = int(ref.tokens.numel())
        differs = (self.tokens[:n] != ref.tokens).nonzero()
        prefix = int(differs[0, 0]) if differs.numel() else n
        return {"gate_token_match": f"{prefix}/{n}", "gate_prefix": prefix,
                "last_logits_max_diff": round(float((self.logits - ref.logits).abs().max()), 4)}


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _generate(model, inputs, n):
    return model.generate(**inputs, do_sample=False, max_new_tokens=n, min_new_tokens=n)


@torch.inference_mode()
def trace(model, inputs, n: int) -> Trace:
    logits = model(**inputs).logits[0, -1].float()
    seq = _generate(model, inputs, n)
    return Trace(seq[0, inputs["input_ids"].shape[1]:], logits)


@torch.inference_mode()
def prefill_seconds(model, inputs, budget_s: float) -> float:
    """Median wall time of one prompt forward, from HIP events around each repeat, after one warmup,
    repeated until ``budget_s`` is spent (at least three repeats)."""
    model(**inputs)
    times, spent = [], 0.0
    while len(times) < 3 or spent < budget_s:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        model(**inputs)
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b) * 1e-3)
        spent += times[-1]
    return statistics.median(times)


@torch.inference_mode()
def decode_rate(model, inputs, n: int, runs: int, prefill_s: float) -> tuple[float, float]:
    """(tokens per second of the decode part, seconds of the fastest generate): n greedy tokens per
    generate, the prompt's prefill time taken out."""
    best = float("inf")
    for _ in range(max(1, runs)):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        _generate(model, inputs, n)
        torch.cuda.synchronize()
        best = min(best, time.perf_counter() - t0)
    return n / max(best - prefill_s, 1e-9), best


def sweep(model, inputs, name: str, variants=None, opts: Options | None = None) -> dict:
    """Measures every variant of SWAPS[name] (stock first) and restores stock at the end."""
    opts = opts or Options()
    swap, known = SWAPS[name]
    order = ["stock"] + [v for v in (known if variants is None else variants) if v != "stock"]
    ref = None
    results = {}
    try:
        for v in order:
            t0 = time.time()
            swap(model, v)
            tr = trace(model, inputs, opts.gate_tokens)
            ref = ref or tr
            p = prefill_seconds(model, inputs, opts.prefill_seconds)
            rate, gen = decode_rate(model, inputs, opts.decode_tokens, opts.decode_runs, p)
            results[v] = {"prefill_ms": round(p * 1e3, 2), "decode_tok_s": round(rate, 2), "generate_s": round(gen, 3),
                          **tr.against(ref), "last_logits_std": round(float(ref.logits.std()), 4)}
            _log(f"{v}: {results[v]} ({time.time() - t0:.0f} s)")
    finally:
        swap(model, "stock")
    return results


def stock_drift(model, inputs, gate_tokens: int) -> dict:
    """The gate's calibration: stock under transformers' other experts implementation (grouped_mm vs
    eager) against stock as configured, by the same two numbers."""
    cfg = getattr(model.config, "text_config", model.config)
    current = cfg._experts_implementation
    other = "eager" if current != "eager" else "grouped_mm"
    base = trace(model, inputs, gate_tokens)
    try:
        model.set_experts_implementation(other)
    except (ValueError, ImportError) as e:  # grouped_mm may not dispatch on this build
        return {"other": other, "error": str(e)}
    try:
        alt = trace(model, inputs, gate_tokens)
    finally:
        model.set_experts_implementation(current)
    return {"other": other, **alt.against(base)}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("model", choices=sorted(SWAPS))
    ap.add_argument("--checkpoint", help="local transformers checkpoint directory (default: seeded random weights)")
    ap.add_argument("--layers", type=int, help="decoder layers (default: the model's)")
    ap.add_argument("--prefill-tokens", type=int, help="prompt length (default: the reference's)")
    ap.add_argument("--decode-tokens", type=int, default=Options.decode_tokens)
    ap.add_argument("--gate-tokens", type=int, default=Options.gate_tokens)
    ap.add_argument("--runs", type=int, default=Options.decode_runs, help="generate runs per variant (best is kept)")
    ap.add_argument("--min-run-time", type=float, default=Options.prefill_seconds,
                    help="seconds of prefill timing per variant")
    ap.add_argument("--variants", help="comma list (stock is always first)")
    ap.add_argument("--stock-experts", choices=["default", "eager", "grouped_mm"], default="default",
                    help="transformers experts implementation of the stock variant")
    ap.add_argument("--out", default="analysis", help="root of the saved results: <out>/<host>/model/<model>.json")
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
    opts = Options(args.gate_tokens, args.decode_tokens, args.runs, args.min_run_time)
    results = sweep(model, inputs, args.model, variants, opts)
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
    out = Path(args.out) / payload["machine"]["host"] / "model"
    out.mkdir(parents=True, exist_ok=True)
    (out / f"{args.model}.json").write_text(json.dumps(payload, indent=1))
    print(json.dumps(payload, indent=1), flush=True)


if __name__ == "__main__":
    main()
