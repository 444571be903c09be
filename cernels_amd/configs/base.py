"""Config: one benchmarkable workload (src/configs/base.py:41-58 of the reference).

The reference's fields, with the same meaning: ``name``, ``dtype``, ``op``, ``inputs(device, dtype)``,
``baseline(*inputs)`` (the reference workload: the transformers module the config stands for, run
eagerly, "op_eager"), ``custom(*inputs)`` (the drop-in loader), ``hub`` / ``lib`` (other contenders;
none here), ``reference_is_hub`` (the baseline is itself a Hub kernel) and ``use_compile`` (also time
``torch.compile(baseline)`` as "op_compile"), and ``verify(out, ref)``.

``use_compile`` is off for every config here: the transformers experts loop is data dependent
(``nonzero`` / ``where`` per hit expert), so compiling it breaks the graph at every expert, and the
reference's own published op_compile times equal its op_eager times within 10%. A config whose
baseline is unavailable offline (the megablocks Hub kernel) has ``baseline = None``; the runner then
times ``custom`` alone.
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
    baseline: Callable[..., Any] | None = None
    hub: Callable[..., Any] | None = None
    lib: Callable[..., Any] | None = None
    reference_is_hub: bool = False
    use_compile: bool = False

    def inputs(self, device, dtype=torch.bfloat16) -> tuple:
        raise NotImplementedError

    def verify(self, out, ref) -> bool:
        # The reference MoE configs' gate (e.g. configs/registry/cohere2_moe_experts.py:89-92).
        return bool(torch.allclose(out.float(), ref.float(), atol=2e-2, rtol=2e-2))
