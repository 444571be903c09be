"""Print the saved benchmark records, one row per (config, machine) (src/benchmark/view.py).

Usage: python -m cernels_amd.benchmark.view [--root DIR]   (default root: analysis)

Columns: each workload's mean ms; each contender's speedup over the reference bar (op_compile if it
ran, else op_eager, else hub); each contender's verdict: "ok" (verified), "FAIL" (verify failed),
"." (ran without a verdict, or declared but did not run), "-" (the config has no such workload). A
declared workload that raised shows "skip" in its ms column (the reason is in the record).
"""

from __future__ import annotations

import argparse
import json
from pathlib import Path

WORKLOADS = ("op_eager", "op_compile", "hub", "lib", "custom")
CONTENDERS = ("hub", "lib", "custom")
BAR = ("op_compile", "op_eager", "hub")


def load(root) -> list[dict]:
    return [json.loads(p.read_text()) for p in sorted(Path(root).glob("*/*.json"))]


def _mark(declared, ran, verified):
    if not declared:
        return "-"
    if not ran or verified is None:
        return "."
    return "ok" if verified else "FAIL"


def rows(records) -> list[list[str]]:
    head = ["config", "gpu", "arch", *(f"{w} ms" for w in WORKLOADS), *(f"{w} vs ref" for w in CONTENDERS),
            *(f"{w} verified" for w in CONTENDERS)]
    out = [head]
    for r in sorted(records, key=lambda r: (r["config"], str(r["machine"].get("gpu")))):
        mean = {w: d["mean_ms"] for w, d in r["workloads"].items()}
        ref = r.get("reference")
        declared = r.get("declared", {})
        bar = next((mean[w] for w in BAR if w in mean), None)
        vs = ["-" if w == ref or bar is None or w not in mean else f"{bar / mean[w]:.2f}x" for w in CONTENDERS]
        ver = ["-" if w == ref else _mark(declared.get(w, False), w in mean, r["workloads"].get(w, {}).get("verified"))
               for w in CONTENDERS]
        mach = r["machine"]
        skipped = r.get("skipped", {})
        ms = [f"{mean[w]:.3f}" if w in mean else ("skip" if w in skipped else "-") for w in WORKLOADS]
        out.append([r["config"], str(mach.get("gpu")), str(mach.get("gcn_arch") or mach.get("arch")), *ms, *vs, *ver])
    return out


def render(table) -> str:
    widths = [max(len(row[i]) for row in table) for i in range(len(table[0]))]
    return "\n".join("  ".join(c.rjust(w) if j > 2 else c.ljust(w) for j, (c, w) in enumerate(zip(row, widths)))
                     for row in table)


def main(root="analysis") -> str:
    recs = load(root)
    text = render(rows(recs)) if recs else f"no results under {root}/ (run python -m cernels_amd.benchmark.main <config>)"
    print(text)
    return text


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--root", default="analysis")
    main(ap.parse_args().root)
