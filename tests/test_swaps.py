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


def _calls(model, T, K=8):
    h = torch.zeros(T, 4)
    idx = torch.zeros(T, K, dtype=torch.int64)
    return [layer["experts"](h, idx, None) for layer in model.layers]


def test_install_dispatch_and_restore():
    m = TinyModel()
    seen = []
    prefill = lambda h, i, w, mod: seen.append(("prefill", h.size(0), mod)) or "p"  # noqa: E731
    decode = lambda h, i, w, mod: seen.append(("decode", h.size(0), mod)) or "d"  # noqa: E731
    assert swaps.install(m, "Cohere2MoeExperts", prefill, decode) == 2
    # the decode GEMV takes every call within its limits: T <= 64 tokens and T*K <= 256 pairs
    assert _calls(m, 32, K=8) == ["d", "d"]
    assert _calls(m, 33, K=8) == ["p", "p"]
    assert _calls(m, 64, K=4) == ["d", "d"]
    assert _calls(m, 65, K=1) == ["p", "p"]
    assert seen[0][2] is m.layers[0]["experts"] and seen[1][2] is m.layers[1]["experts"]
    swaps.install(m, "Cohere2MoeExperts", prefill, None)  # prefill only: the reference's 4-token switch
    assert _calls(m, 1) == [("stock", 1)] * 2
    assert _calls(m, 4) == [("stock", 4)] * 2
    assert _calls(m, 5) == ["p", "p"]  # above 4 tokens, even where the decode GEMV would take the call
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

    c = rand_case(21, 160, 256, 128, 8, 2)
    m = TinyModel(n=1, gate_up_proj=c["W1"], down_proj=c["W2"]).to(device)
    swaps.north_mini_code(m, "custom")
    ex = m.layers[0]["experts"]
    assert swaps.use_decode(3, 2) and not swaps.use_decode(160, 2)
    for rows in (slice(0, 3), slice(None)):  # decode entry, then prefill entry (160 tokens x 2 slots > 256 pairs)
        out = ex(c["x"][rows].to(device), c["idx"][rows].to(device), c["w"][rows].to(device))
        ref = O.experts_fp64(c["x"][rows], c["idx"][rows], c["w"][rows], c["W1"], c["W2"])
        assert_within_tolerance(out.cpu(), ref, f"swapped rows {rows}")


# ---- whole-model runner (cernels_amd.modeling.main) on the real transformers architectures ----

_TINY_NMC = dict(hidden_size=128, num_attention_heads=4, num_key_value_heads=2, head_dim=32, intermediate_size=64,
                 prefix_dense_intermediate_size=256, num_experts=8, vocab_size=1000)
_TINY_DS = dict(hidden_size=128, intermediate_size=256, moe_intermediate_size=64, num_attention_heads=4,
                num_key_value_heads=4, n_routed_experts=8, num_experts_per_tok=2, vocab_size=1000)


def test_model_configs_match_the_documented_architectures():
    from cernels_amd.modeling import models as M

    c = M.make_config(M.NORTH_MINI_CODE)
    assert (c.num_hidden_layers, c.hidden_size, c.intermediate_size, c.num_experts, c.num_experts_per_tok) == \
        (49, 2048, 768, 128, 8)
    assert c.mlp_layer_types[0] == "dense" and set(c.mlp_layer_types[1:]) == {"sparse"}
    assert (c.num_attention_heads, c.num_key_value_heads, c.head_dim, c.sliding_window) == (32, 4, 128, 4096)
    assert c.expert_selection_fn == "sigmoid" and c.norm_topk_prob is False and c.num_shared_experts == 0
    d = M.make_config(M.DEEPSEEK_OCR_2).text_config
    assert (d.num_hidden_layers, d.hidden_size, d.moe_intermediate_size, d.n_routed_experts, d.num_experts_per_tok,
            d.n_shared_experts) == (12, 1280, 896, 64, 6, 2)
    assert d.mlp_layer_types[0] == "dense" and set(d.mlp_layer_types[1:]) == {"sparse"}


@pytest.mark.parametrize("name,tiny,cls", [("north_mini_code", _TINY_NMC, "Cohere2MoeExperts"),
                                           ("deepseek_ocr_2", _TINY_DS, "DeepseekOcr2TextExperts")])
def test_swap_targets_every_moe_layer_of_the_real_model(name, tiny, cls):
    from cernels_amd.modeling import models as M

    model = M.build(M.SPECS[name], device="cpu", layers=3, **tiny)
    n = sum(type(m).__name__ == cls for m in model.modules())
    assert n == 2  # layer 0 is dense
    fn, variants = swaps.SWAPS[name]
    assert fn(model, variants[-1]) == n
    assert all("forward" in vars(m) for m in model.modules() if type(m).__name__ == cls)
    fn(model, "stock")
    assert not any("forward" in vars(m) for m in model.modules() if type(m).__name__ == cls)


@pytest.mark.gpu
@pytest.mark.parametrize("name,tiny", [("north_mini_code", _TINY_NMC), ("deepseek_ocr_2", _TINY_DS)])
def test_whole_model_runner_on_a_small_model(device, name, tiny):
    """Every variant runs end to end through generate(); the swapped model's last prefill logits stay
    close to stock (bf16 model, fp32-accumulating experts)."""
    from cernels_amd.modeling import main as runner
    from cernels_amd.modeling import models as M

    spec = M.SPECS[name]
    model = M.build(spec, device="cuda", layers=3, **tiny)
    inputs = M.prompt_ids(spec, 40, "cuda", vocab=1000)
    print(f"[whole model {name}]", flush=True)
    opts = runner.Options(gate_tokens=6, decode_tokens=6, decode_runs=1, prefill_seconds=0.05)
    res = runner.sweep(model, inputs, name, opts=opts)
    _, variants = swaps.SWAPS[name]
    assert list(res) == list(variants)
    stock = runner.trace(model, inputs, 1).logits
    for v in variants[1:]:
        swaps.SWAPS[name][0](model, v)
        lv = runner.trace(model, inputs, 1).logits
        assert float((lv - stock).abs().max()) <= 0.05 * float(stock.abs().max()) + 1e-3, v
        assert res[v]["decode_tok_s"] > 0
    swaps.SWAPS[name][0](model, "stock")


@pytest.mark.gpu
def test_swapped_model_tracks_fp32_as_closely_as_stock(device):
    """The whole-model gate with its drift calibration as a check: an 8-layer north_mini_code
    (Cohere2Moe, real hidden/expert shapes, seeded random weights) run in bf16 three ways — stock
    grouped_mm, stock eager, swapped to this library (prefill and decode kernels) — is compared with
    the same model in float32 (eager experts). The swapped model's greedy continuation must agree with
    the float32 one for at least as many tokens as the worse of transformers' two bf16
    implementations does, and its last prefill logits must be no further from float32's than 1.25x
    the further of the two."""
    import copy

    from cernels_amd.modeling import main as runner
    from cernels_amd.modeling import models as M

    spec = M.SPECS["north_mini_code"]
    model = M.build(spec, device="cuda", layers=8, vocab_size=32000)
    inputs = M.prompt_ids(spec, 300, "cuda", vocab=32000)
    n = 32
    print("[fp32 gate] building the float32 copy", flush=True)
    ref32 = copy.deepcopy(model).float()
    ref32.set_experts_implementation("eager")
    ref = runner.trace(ref32, inputs, n)
    del ref32
    torch.cuda.empty_cache()
    got = {}
    for impl in ("grouped_mm", "eager"):
        model.set_experts_implementation(impl)
        got[f"stock_{impl}"] = runner.trace(model, inputs, n).against(ref)
    model.set_experts_implementation("grouped_mm")
    swaps.SWAPS["north_mini_code"][0](model, "custom")
    try:
        got["custom"] = runner.trace(model, inputs, n).against(ref)
    finally:
        swaps.SWAPS["north_mini_code"][0](model, "stock")
    print(f"[fp32 gate] {got}", flush=True)
    stock = [got["stock_grouped_mm"], got["stock_eager"]]
    assert got["custom"]["gate_prefix"] >= min(s["gate_prefix"] for s in stock), got
    assert got["custom"]["last_logits_max_diff"] <= 1.25 * max(s["last_logits_max_diff"] for s in stock), got


def test_whole_model_results_table(tmp_path):
    """modeling.view tabulates <root>/<host>/model/<model>.json, one row per variant."""
    import json

    from cernels_amd.modeling import view

    d = tmp_path / "box" / "model"
    d.mkdir(parents=True)
    rec = {"model": "north_mini_code", "machine": {"gpu": "gfx950 test", "host": "box"},
           "variants": {"stock": {"prefill_ms": 254.71, "decode_tok_s": 40.1, "generate_s": 3.2,
                                  "gate_token_match": "64/64", "last_logits_max_diff": 0.0},
                        "custom": {"prefill_ms": 51.12, "decode_tok_s": 51.8, "generate_s": 2.5,
                                   "gate_token_match": "0/64", "last_logits_max_diff": 0.135}}}
    (d / "north_mini_code.json").write_text(json.dumps(rec))
    table = view.rows(tmp_path)
    assert [r[2] for r in table[1:]] == ["stock", "custom"]
    assert table[2][3:] == ["51.1", "51.80", "2.50", "0/64", "0.135"]
    assert "north_mini_code" in view.main(tmp_path)
    assert "no whole-model results" in view.main(tmp_path / "none")


def test_decode_limits_are_the_librarys():
    """The swap's dispatch limits are the decode entry's own (host-side queries, no GPU call)."""
    from cernels_amd import _native

    L = _native.lib()
    assert swaps.DECODE_MAX_TOKENS == L.cernels_moe_decode_max_tokens()
    assert swaps.DECODE_MAX_PAIRS == L.cernels_moe_decode_max_pairs()
