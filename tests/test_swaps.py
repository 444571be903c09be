"""Expert-swap dispatch (cernels_amd.modeling.swaps) and the registry loaders.

CPU: the swap installs and removes instance forwards, dispatches by token count and rejects
models without the experts class — with stand-in ops, no GPU calls.
GPU: a swapped experts module gives the oracle's answer through both entry points.
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from cernels_amd.modeling import swaps


class Cohere2MoeExperts(nn.Module):  # same class name as the transformers module the swap targets
    def __init__(self, gate_up_proj=None, down_proj=None):
        super().__init__()
        self.gate_up_proj = None if gate_up_proj is None else nn.Parameter(gate_up_proj, requires_grad=False)
        self.down_proj = None if down_proj is None else nn.Parameter(down_proj, requires_grad=False)

    def forward(self, hidden, top_k_index, top_k_weights):
        return ("stock", hidden.size(0))


class TinyModel(nn.Module):
    def __init__(self, n=2, **kw):
        super().__init__()
        self.layers = nn.ModuleList([nn.ModuleDict({"experts": Cohere2MoeExperts(**kw)}) for _ in range(n)])


def _calls(model, T):
    h = torch.zeros(T, 4)
    return [layer["experts"](h, None, None) for layer in model.layers]


def test_install_dispatch_and_restore():
    m = TinyModel()
    seen = []
    prefill = lambda h, i, w, mod: seen.append(("prefill", h.size(0), mod)) or "p"  # noqa: E731
    decode = lambda h, i, w, mod: seen.append(("decode", h.size(0), mod)) or "d"  # noqa: E731
    assert swaps.install(m, "Cohere2MoeExperts", prefill, decode) == 2
    assert _calls(m, swaps.DECODE_MAX_TOKENS) == ["d", "d"]
    assert _calls(m, swaps.DECODE_MAX_TOKENS + 1) == ["p", "p"]
    assert seen[0][2] is m.layers[0]["experts"] and seen[1][2] is m.layers[1]["experts"]
    swaps.install(m, "Cohere2MoeExperts", prefill, None)  # prefill only: decode-sized calls stay stock
    assert _calls(m, 1) == [("stock", 1)] * 2
    assert _calls(m, 100) == ["p", "p"]
    swaps.install(m, "Cohere2MoeExperts", None, None)  # restore
    assert "forward" not in vars(m.layers[0]["experts"])
    assert _calls(m, 100) == [("stock", 100)] * 2


def test_wrong_model_and_unknown_variant():
    with pytest.raises(RuntimeError, match="no DeepseekOcr2TextExperts"):
        swaps.install(TinyModel(), "DeepseekOcr2TextExperts", lambda *a: None, None)
    with pytest.raises(KeyError):
        swaps.entry_points("north_mini_code", "custom_full")


def test_variants_select_entry_points():
    from cernels_amd.kops.registry import cohere2_moe_experts as c2

    assert swaps.entry_points("north_mini_code", "stock") == (None, None)
    assert swaps.entry_points("north_mini_code", "custom_prefill") == (c2.kernel, None)
    assert swaps.entry_points("north_mini_code", "custom") == (c2.kernel, c2.decode_kernel)
    fn, variants = swaps.SWAPS["north_mini_code"]
    assert variants[0] == "stock" and callable(fn)


@pytest.mark.gpu
def test_swapped_module_matches_oracle(device):
    from helpers import assert_within_tolerance, rand_case
    from oracle import eager as O

    c = rand_case(21, 40, 256, 128, 8, 2)
    m = TinyModel(n=1, gate_up_proj=c["W1"], down_proj=c["W2"]).to(device)
    swaps.north_mini_code(m, "custom")
    ex = m.layers[0]["experts"]
    for rows in (slice(0, 3), slice(None)):  # decode entry, then prefill entry
        out = ex(c["x"][rows].to(device), c["idx"][rows].to(device), c["w"][rows].to(device))
        ref = O.experts_fp64(c["x"][rows], c["idx"][rows], c["w"][rows], c["W1"], c["W2"])
        assert_within_tolerance(out.cpu(), ref, f"swapped rows {rows}")
