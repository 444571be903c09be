"""Persistence: one record per config and machine, ``<root>/<host>/<config>.json`` plus the run's log
(src/benchmark/save.py; the latest run per machine replaces the previous one)."""

from __future__ import annotations

import hashlib
import json
import platform
import socket
from dataclasses import asdict, is_dataclass
from datetime import datetime
from pathlib import Path

import torch

ANALYSIS = Path("analysis")
CSRC = Path(__file__).resolve().parents[1] / "csrc"


def machine() -> dict:
    rec = {"gpu": None, "gcn_arch": None, "arch": platform.machine(), "backend": f"ROCm/HIP {torch.version.hip}",
           "torch": torch.__version__, "os": f"{platform.system()} {platform.release()}", "host": socket.gethostname()}
    if torch.cuda.is_available():
        p = torch.cuda.get_device_properties(0)
        rec["gpu"], rec["gcn_arch"] = p.name, getattr(p, "gcnArchName", None)
    return rec


def input_shapes(cfg) -> list:
    """Shapes of the config's tensor inputs, from meta tensors (nothing is allocated)."""
    try:
        return [list(t.shape) for t in cfg.inputs("meta", cfg.dtype) if hasattr(t, "shape")]
    except Exception:  # a module-level config builds modules, not meta tensors
        return []


def library_sha() -> str:
    """Short SHA-256 over the native sources (file names and contents, sorted): what the custom
    workload's performance is built from."""
    h = hashlib.sha256()
    for f in sorted(CSRC.glob("*")):
        if f.suffix in (".hip", ".cpp", ".h"):
            h.update(f.name.encode())
            h.update(f.read_bytes())
    return h.hexdigest()[:12]


def record(name, cfg, results, ref_label, skipped=None) -> dict:
    declared = {
        "op_eager": cfg.baseline is not None and not cfg.reference_is_hub,
        "op_compile": cfg.baseline is not None and not cfg.reference_is_hub and cfg.use_compile,
        "hub": cfg.reference_is_hub or cfg.hub is not None,
        "lib": cfg.lib is not None,
        "custom": cfg.custom is not None,
    }
    return {
        "timestamp": datetime.now().isoformat(timespec="seconds"),
        "config": name,
        "op": cfg.op,
        "dtype": str(cfg.dtype).removeprefix("torch."),
        "input_shapes": input_shapes(cfg),
        "machine": machine(),
        "reference": ref_label,
        "declared": declared,
        "provenance": {"repo": None, "version": None, "kernel_commit_sha": None, "custom_sha": library_sha()},
        "workloads": {w: asdict(t) if is_dataclass(t) else dict(t) for w, t in results.items()},
        "skipped": dict(skipped or {}),  # declared workloads that raised, with the reason
    }


def save(name, cfg, results, log, ref_label="op_eager", root=ANALYSIS, skipped=None) -> Path:
    rec = record(name, cfg, results, ref_label, skipped)
    out = Path(root) / rec["machine"]["host"]
    out.mkdir(parents=True, exist_ok=True)
    path = out / f"{name}.json"
    path.write_text(json.dumps(rec, indent=2))
    (out / f"{name}.log").write_text(log)
    return path
