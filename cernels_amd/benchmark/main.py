"""Time one config's workloads under the reference's benchmark protocol (src/benchmark/main.py:20-63).

Usage: python -m cernels_amd.benchmark.main <config> [--root DIR] [--only LABEL ...]
       (<config> = a key of cernels_amd.configs.registry.CONFIGS)

The protocol, as the reference defines it: the reference workload is op_eager (the transformers module
the config stands for), or hub when the config's baseline is itself a Hub kernel; op_compile is
``torch.compile`` of that baseline when the config asks for it; hub / lib / custom are contenders.
Every workload gets 10 untimed calls, one call whose output is checked against the reference's output
with the config's ``verify`` (not for the reference itself), and ``blocked_autorange`` sampling with a
1 s budget. The record goes to ``<root>/<host>/<config>.json`` with the run's log beside it.

How this module is built: a config becomes a *lineup* of ``Entrant``s. A ``Bench`` holds the inputs,
the reference output and the reference mean, and takes each entrant through three phases (``prime``,
``check``, ``sample``). A phase that raises does not end the run: the entrant is recorded under
``skipped`` with the reason, and that dictionary is part of the saved record (a compile that fails on a
data-dependent op shows up there, not only in the log).
"""

from __future__ import annotations

import argparse
import sys
from dataclasses import dataclass, field
from typing import Any, Callable

import torch
from torch.utils.benchmark import Timer

from cernels_amd.benchmark.monitor import TimingResults, capture, stats
from cernels_amd.benchmark.save import ANALYSIS, save

WARMUP_CALLS = 10   # protocol: untimed calls before sampling (src/benchmark/main.py:20)
SAMPLE_BUDGET_S = 1.0  # protocol: blocked_autorange budget per workload (src/benchmark/main.py:21)
LABELS = ("op_eager", "op_compile", "hub", "lib", "custom")


@dataclass(frozen=True)
class Entrant:
    label: str
    call: Callable[..., Any]
    is_reference: bool = False


def _compiled_baseline(cfg):
    return torch.compile(cfg.baseline)


def lineup(cfg) -> list[Entrant]:
    """The config's workloads in protocol order, the reference first (none when the baseline is absent,
    e.g. a Hub kernel that needs the network)."""
    out: list[Entrant] = []
    eager_reference = cfg.baseline is not None and not cfg.reference_is_hub
    if cfg.baseline is not None:
        out.append(Entrant("op_eager" if eager_reference else "hub", cfg.baseline, is_reference=True))
    # each contender slot: (label, is it declared, how to get its callable)
    slots = (("op_compile", eager_reference and cfg.use_compile, lambda: _compiled_baseline(cfg)),
             ("hub", cfg.hub is not None and not cfg.reference_is_hub, lambda: cfg.hub),
             ("lib", cfg.lib is not None, lambda: cfg.lib),
             ("custom", cfg.custom is not None, lambda: cfg.custom))
    out.extend(Entrant(label, get()) for label, declared, get in slots if declared)
    return out


def _tensor_of(result):
    """The tensor an output is verified by: the result itself, or the first element of a tuple/list."""
    while isinstance(result, (tuple, list)):
        result = result[0]
    return result


def _device_sync(device) -> None:
    if torch.device(device).type == "cuda":
        torch.cuda.synchronize()


@dataclass
class Outcome:
    results: dict[str, TimingResults] = field(default_factory=dict)
    reference: str | None = None
    skipped: dict[str, str] = field(default_factory=dict)


class Bench:
    """One config's inputs on one device, and the reference's output and mean once measured."""

    def __init__(self, cfg, device="cuda", warmup=WARMUP_CALLS, budget_s=SAMPLE_BUDGET_S):
        self.cfg, self.device, self.warmup, self.budget_s = cfg, device, warmup, budget_s
        self.args = cfg.inputs(device, cfg.dtype)
        self.expected = None      # the reference's output tensor
        self.reference_ms = None  # the reference's mean

    def prime(self, e: Entrant) -> None:
        for _ in range(self.warmup):
            e.call(*self.args)
        _device_sync(self.device)

    def check(self, e: Entrant) -> bool | None:
        if e.is_reference or self.expected is None:
            return None
        return bool(self.cfg.verify(_tensor_of(e.call(*self.args)), self.expected))

    def sample(self, e: Entrant) -> tuple[list[float], int]:
        timer = Timer(stmt="call(*args)", globals={"call": e.call, "args": self.args})
        m = timer.blocked_autorange(min_run_time=self.budget_s)
        return [1e3 * t for t in m.times], m.number_per_run

    def measure(self, e: Entrant) -> TimingResults:
        print(f"  {e.label}: {self.warmup} untimed calls", file=sys.stderr)  # a compile happens in these
        self.prime(e)
        verdict = self.check(e)
        times, per_block = self.sample(e)
        print(f"  {e.label}: {len(times)} blocks of {per_block} calls", file=sys.stderr)
        res = stats(times, verdict, None if e.is_reference else self.reference_ms)
        if e.is_reference:
            self.reference_ms = res.mean_ms
        return res


def run(cfg, device="cuda", warmup=WARMUP_CALLS, budget_s=SAMPLE_BUDGET_S, only=None) -> Outcome:
    """Measures each entrant of ``cfg`` (or those whose labels are in ``only``; the reference's output is
    computed regardless, so contenders are still verified)."""
    bench = Bench(cfg, device, warmup, budget_s)
    entrants = lineup(cfg)
    outcome = Outcome(reference=next((e.label for e in entrants if e.is_reference), None))
    with torch.no_grad():
        for e in entrants:
            if e.is_reference:
                bench.expected = _tensor_of(e.call(*bench.args))
            if only is not None and e.label not in only:
                continue
            try:
                outcome.results[e.label] = bench.measure(e)
            except Exception as exc:  # recorded, and the remaining entrants still run
                reason = f"{type(exc).__name__}: {exc}".splitlines()[0][:400]
                outcome.skipped[e.label] = reason
                print(f"  {e.label}: skipped ({reason})", file=sys.stderr)
    return outcome


def table(outcome: Outcome) -> str:
    head = ("workload", "mean ms", "std", "min", "max", "samples", "speedup", "verify")
    body = []
    for label, r in outcome.results.items():
        verdict = "-" if r.verified is None else ("pass" if r.verified else "FAIL")
        body.append((label, f"{r.mean_ms:.4f}", f"{r.std_ms:.4f}", f"{r.min_ms:.4f}", f"{r.max_ms:.4f}",
                     str(r.iterations), "-" if r.speedup is None else f"{r.speedup:.2f}x", verdict))
    body.extend((label, "skipped", "", "", "", "", "", "") for label in outcome.skipped)
    widths = [max(len(row[i]) for row in (head, *body)) for i in range(len(head))]
    return "\n".join("  ".join(c.ljust(w) for c, w in zip(row, widths)) for row in (head, *body))


def main(name, root=ANALYSIS, device="cuda", only=None) -> Outcome:
    from cernels_amd.configs.registry import CONFIGS

    cfg = CONFIGS.get(name)
    if cfg is None:
        raise SystemExit(f"unknown config {name!r}; one of: {', '.join(sorted(CONFIGS))}")
    with capture() as log:
        print(f"[{name}] {cfg.op}", file=sys.stderr)
        outcome = run(cfg, device, only=only)
        print(table(outcome), file=sys.stderr)
    path = save(name, cfg, outcome.results, log.getvalue(), ref_label=outcome.reference, root=root,
                skipped=outcome.skipped)
    print(f"wrote {path}", file=sys.stderr)
    return outcome


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("config")
    ap.add_argument("--root", default=str(ANALYSIS), help="directory of the saved records (default: analysis)")
    ap.add_argument("--only", nargs="+", choices=LABELS, help="measure only these workloads")
    args = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit("the benchmark runs on a GPU")
    main(args.config, root=args.root, only=args.only)
