"""Config: one benchmarkable workload (src/configs/base.py:41-58 of the reference).

Fields kept from the reference: ``name``, ``dtype``, ``op``, ``inputs(device, dtype)``, ``custom``
and ``verify(out, ref)``. The reference's ``baseline`` calls the transformers module; here the
op_eager restatement lives with the test-side checker, so a Config carries only the shape and how
to build its inputs.
"""

from __future__ import annotations

from collections.abc import Callable
from typing import Any

import torch

from cernels_amd.configs.synth import MoeShape


class Config:
    name: str = ""
    dtype: torch.dtype = torch.bfloat16
    op: str = ""
    shape: MoeShape
    custom: Callable[..., Any] | None = None

    def inputs(self, device, dtype=torch.bfloat16) -> tuple:
        raise NotImplementedError

    def verify(self, out, ref) -> bool:
        # The reference MoE configs' gate (e.g. configs/registry/cohere2_moe_experts.py:89-92).
        return bool(torch.allclose(out.float(), ref.float(), atol=2e-2, rtol=2e-2))
