"""Tabulate saved whole-model results, one row per (model, machine, variant) (src/modeling/view.py).

Usage: python -m cernels_amd.modeling.view [--root DIR]   (reads <root>/<host>/model/<model>.json; default
root: analysis, where ``python -m cernels_amd.modeling.main`` writes them)
"""

from __future__ import annotations

import argparse
import json
from pathlib import Path

COLS = ("model", "gpu", "variant", "prefill ms", "decode tok/s", "generate s", "greedy match", "logits max diff")


def rows(root) -> list[list[str]]:
    out = [list(COLS)]
    for path in sorted(Path(root).glob("*/model/*.json")):
        r = json.loads(path.read_text())
        for variant, v in r["variants"].items():
            out.append([r["model"], str(r["machine"]["gpu"]), variant, f"{v['prefill_ms']:.1f}",
                        f"{v['decode_tok_s']:.2f}", f"{v['generate_s']:.2f}", v["gate_token_match"],
                        f"{v['last_logits_max_diff']:.3f}"])
    return out


def main(root="analysis") -> str:
    table = rows(root)
    if len(table) == 1:
        text = f"no whole-model results under {root}/*/model/ (run python -m cernels_amd.modeling.main <model>)"
    else:
        widths = [max(len(row[i]) for row in table) for i in range(len(COLS))]
        text = "\n".join("  ".join(c.rjust(w) if j > 2 else c.ljust(w) for j, (c, w) in enumerate(zip(row, widths)))
                         for row in table)
    print(text)
    return text


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--root", default="analysis")
    main(ap.parse_args().root)
