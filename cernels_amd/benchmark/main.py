"""Benchmark a config's workloads (src/benchmark/main.py): the reference (op_eager: the transformers
module the config stands for) and the contenders (custom: this library's drop-in loader).

Usage: python -m cernels_amd.benchmark.main <config> [--root DIR]
       (<config> = a key of cernels_amd.configs.registry.CONFIGS)

Per workload: 10 untimed calls, one more call checked against the reference's output with the
config's ``verify`` (contenders only), then ``torch.utils.benchmark.Timer.blocked_autorange`` with a
1 s budget; per-iteration times are reduced to statistics. The record goes to
``<root>/<host>/<config>.json`` with the run's log beside it (root ``analysis`` by default).
"""

from __future__ import annotations

import argparse
import sys

import torch
from torch.utils.benchmark import Timer

from cernels_amd.benchmark.monitor import capture, stats
from cernels_amd.benchmark.save import ANALYSIS, save

WARMUP = 10       # src/benchmark/main.py:20
MIN_RUN_S = 1.0   # src/benchmark/main.py:21


def _first(out):
    """The output tensor of a workload (module-level ops may return a tuple)."""
    return out[0] if isinstance(out, (tuple, list)) else out


def workloads(cfg) -> tuple[dict, str | None]:
    """(name -> callable, the reference's name). The reference is op_eager, or hub when the config's
    baseline is a Hub kernel; a config without a baseline here (a Hub reference, offline) has none."""
    ref_label = None
    wl = {}
    if cfg.baseline is not None:
        ref_label = "hub" if cfg.reference_is_hub else "op_eager"
        wl[ref_label] = cfg.baseline
        if not cfg.reference_is_hub and cfg.use_compile:
            wl["op_compile"] = torch.compile(cfg.baseline)
    if cfg.hub is not None and ref_label != "hub":
        wl["hub"] = cfg.hub
    if cfg.lib is not None:
        wl["lib"] = cfg.lib
    if cfg.custom is not None:
        wl["custom"] = cfg.custom
    return wl, ref_label


def run(cfg, device="cuda", warmup=WARMUP, min_run_s=MIN_RUN_S):
    """Times every workload of ``cfg`` on its own inputs; returns ({workload: TimingResults}, reference)."""
    inputs = cfg.inputs(device, cfg.dtype)
    wl, ref_label = workloads(cfg)
    results, ref = {}, None
    with torch.no_grad():
        if ref_label is not None:
            ref = _first(wl[ref_label](*inputs))
        ref_mean = None
        for name, fn in wl.items():
            try:
                for _ in range(warmup):
                    fn(*inputs)
                torch.cuda.synchronize()
                verified = None if name == ref_label or ref is None else bool(cfg.verify(_first(fn(*inputs)), ref))
                m = Timer(stmt="fn(*inputs)", globals={"fn": fn, "inputs": inputs}).blocked_autorange(
                    min_run_time=min_run_s)
            except Exception as exc:  # one failing workload does not end the run
                print(f"  {name}: skipped ({type(exc).__name__}: {exc})", file=sys.stderr)
                continue
            times = [t * 1e3 for t in m.times]
            print(f"  {name}: {len(times)} samples x {m.number_per_run} iterations", file=sys.stderr)
            results[name] = stats(times, verified, None if name == ref_label else ref_mean)
            if name == ref_label:
                ref_mean = results[name].mean_ms
    return results, ref_label


def table(results) -> str:
    rows = [("workload", "mean ms", "std", "min", "max", "n", "vs ref", "verified")]
    for name, r in results.items():
        rows.append((name, f"{r.mean_ms:.4f}", f"{r.std_ms:.4f}", f"{r.min_ms:.4f}", f"{r.max_ms:.4f}",
                     str(r.iterations), "-" if r.speedup is None else f"{r.speedup:.2f}x",
                     "-" if r.verified is None else ("yes" if r.verified else "NO")))
    widths = [max(len(row[i]) for row in rows) for i in range(len(rows[0]))]
    return "\n".join("  ".join(c.ljust(w) for c, w in zip(row, widths)) for row in rows)


def main(name, root=ANALYSIS, device="cuda"):
    from cernels_amd.configs.registry import CONFIGS

    if name not in CONFIGS:
        raise SystemExit(f"unknown config {name!r}; one of: {', '.join(sorted(CONFIGS))}")
    cfg = CONFIGS[name]
    with capture() as log:
        print(f"[{name}] {cfg.op}", file=sys.stderr)
        results, ref_label = run(cfg, device)
        print(table(results), file=sys.stderr)
    path = save(name, cfg, results, log.getvalue(), ref_label=ref_label, root=root)
    print(f"wrote {path}", file=sys.stderr)
    return results


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("config")
    ap.add_argument("--root", default=str(ANALYSIS), help="directory of the saved records (default: analysis)")
    args = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit("the benchmark runs on a GPU")
    main(args.config, root=args.root)
