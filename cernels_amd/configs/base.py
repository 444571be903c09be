"""Config: one benchmarkable workload (src/configs/base.py:41-58 of the reference).

The reference's fields, with the same meaning: ``name``, ``dtype``, ``op``, ``inputs(device, dtype)``,
``baseline(*inputs)`` (the reference workload: the transformers module the config stands for, run
eagerly, "op_eager"), ``custom(*inputs)`` (the drop-in loader), ``hub`` / ``lib`` (other contenders;
none here), ``reference_is_hub`` (the baseline is itself a Hub kernel) and ``use_compile`` (also time
``torch.compile(baseline)`` as "op_compile"), and ``verify(out, ref)``.

``use_compile`` is on, as in the reference's MoE configs (src/configs/registry/cohere2_moe_experts.py:30,
deepseek_ocr2_moe_experts.py:33, gpt_oss_moe_experts.py:27, qwen3_next_moe_experts.py:39). The
transformers experts loop is data dependent (``nonzero`` / ``where`` per hit expert), so the compiled
baseline runs as many small graphs with breaks between them; where compiling fails the runner records
op_compile as skipped, with the reason. A config whose baseline is unavailable offline (the megablocks
Hub kernel) has ``baseline = None`` and ``use_compile`` off (src/configs/registry/megablocks_moe.py:21-22);
the runner then times ``custom`` alone.
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
    use_compile: bool = True

    def inputs(self, device, dtype=torch.bfloat16) -> tuple:
        raise NotImplementedError

    def verify(self, out, ref) -> bool:
        # The reference MoE configs' gate (e.g. configs/registry/cohere2_moe_experts.py:89-92).
        return bool(torch.allclose(out.float(), ref.float(), atol=2e-2, rtol=2e-2))
