"""Shared test configuration.

Markers: ``gpu`` — needs an MI355X (HIP device) and the built native library. Everything else
runs on the CPU. The oracle (oracle/) is the checker; the product path is cernels_amd.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built libcernels_moe.so")


def gpu_available() -> bool:
    return torch.cuda.is_available()


def load_golden(name: str):
    from safetensors import safe_open
    from safetensors.torch import load_file

    path = GOLDEN / f"{name}.safetensors"
    tensors = load_file(str(path))
    with safe_open(str(path), framework="pt") as f:
        meta = json.loads(f.metadata()["meta"])
    return tensors, meta


GOLDEN_NAMES = sorted(p.stem for p in GOLDEN.glob("*.safetensors"))


@pytest.fixture(scope="session")
def device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cernels_amd import _native

    _native.lib()  # fail loudly (not skip) when the native library is missing on a GPU box
    return torch.device("cuda:0")
