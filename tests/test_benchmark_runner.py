"""The benchmark runner (cernels_amd.benchmark, the reference's src/benchmark/): statistics, the saved
record, the results table, and each config's op_eager baseline. The GPU test runs one reference config
end to end."""

from __future__ import annotations

import json

import pytest
import torch

from cernels_amd.benchmark import main as runner
from cernels_amd.benchmark import monitor, save, view


def test_stats_quartiles_and_tukey_outliers():
    # 1..9 and one far sample: q1/q3 by linear interpolation between closest ranks (numpy's default)
    t = [1.0, 2, 3, 4, 5, 6, 7, 8, 9, 100]
    r = monitor.stats(t, verified=True, ref_mean_ms=29.0)
    assert r.iterations == 10 and r.min_ms == 1.0 and r.max_ms == 100.0
    assert r.mean_ms == pytest.approx(14.5)
    assert r.std_ms == pytest.approx((sum((x - 14.5) ** 2 for x in t) / 10) ** 0.5, abs=1e-4)
    assert (r.q1_ms, r.q3_ms) == (pytest.approx(3.25), pytest.approx(7.75))
    assert r.outliers == 1  # only 100 lies beyond q3 + 1.5 IQR = 14.5
    assert r.speedup == pytest.approx(2.0) and r.verified is True
    one = monitor.stats([2.5])
    assert (one.mean_ms, one.std_ms, one.iqr_ms, one.outliers, one.speedup) == (2.5, 0.0, 0.0, 0, None)
    with pytest.raises(ValueError):
        monitor.stats([])


def test_capture_echoes_and_keeps_stderr(capsys):
    import sys

    with monitor.capture() as buf:
        print("inside", file=sys.stderr)
    assert buf.getvalue() == "inside\n"
    assert "inside" in capsys.readouterr().err


def test_saved_record_and_table(tmp_path):
    from cernels_amd.configs.registry import CONFIGS

    cfg = CONFIGS["cohere2_moe_experts"]
    results = {"op_eager": monitor.stats([4.0, 4.2, 4.1]),
               "custom": monitor.stats([0.10, 0.11, 0.10], verified=True, ref_mean_ms=4.1)}
    path = save.save("cohere2_moe_experts", cfg, results, "log text\n", ref_label="op_eager", root=tmp_path)
    rec = json.loads(path.read_text())
    assert path.parent.parent == tmp_path and path.with_suffix(".log").read_text() == "log text\n"
    assert rec["config"] == "cohere2_moe_experts" and rec["reference"] == "op_eager" and rec["dtype"] == "bfloat16"
    assert rec["declared"] == {"op_eager": True, "op_compile": True, "hub": False, "lib": False, "custom": True}
    assert rec["skipped"] == {}
    s = cfg.shape
    assert rec["input_shapes"] == [[s.tokens, s.hidden], [s.tokens, s.top_k], [s.tokens, s.top_k]]
    assert len(rec["provenance"]["custom_sha"]) == 12
    assert rec["workloads"]["custom"]["verified"] is True and rec["workloads"]["custom"]["speedup"] == pytest.approx(4.1 / 0.10333, rel=1e-3)
    table = view.rows(view.load(tmp_path))
    assert table[1][0] == "cohere2_moe_experts"
    head = table[0]
    assert table[1][head.index("op_eager ms")] == "4.100" and table[1][head.index("op_compile ms")] == "-"
    assert table[1][head.index("custom vs ref")] == "39.69x" and table[1][head.index("custom verified")] == "ok"
    assert table[1][head.index("hub verified")] == "-"
    assert "cohere2_moe_experts" in view.main(tmp_path)
    assert "no results" in view.main(tmp_path / "empty")


def test_lineup_follows_the_protocol_order():
    from cernels_amd.configs.registry import CONFIGS

    assert [e.label for e in runner.lineup(CONFIGS["megablocks_moe"])] == ["custom"]  # its reference is offline
    for name in ("cohere2_moe_experts", "deepseek_ocr2_moe_experts_decode", "gpt_oss_moe_experts", "qwen3_next_moe_experts"):
        ent = runner.lineup(CONFIGS[name])
        assert [e.label for e in ent] == ["op_eager", "op_compile", "custom"], name
        assert [e.is_reference for e in ent] == [True, False, False]


def _small_experts_config():
    from cernels_amd.configs.registry import ExpertsConfig
    from cernels_amd.configs.synth import MoeShape

    cfg = ExpertsConfig(MoeShape("cohere2_small", tokens=9, hidden=64, ffn=32, experts=8, top_k=2))
    cfg.custom = cfg.baseline  # a contender that is the reference itself: verifies, speedup about 1
    return cfg


def test_run_records_each_workload_and_the_skips(monkeypatch, tmp_path):
    """On the CPU with a stand-in compile: the reference is measured first, contenders are verified
    against its output and get a speedup; a workload that raises is recorded under ``skipped`` (in the
    outcome and the saved record) and the run goes on."""
    cfg = _small_experts_config()

    def broken_compile(c):
        def call(*args):
            raise RuntimeError("compile failed on purpose\nsecond line")
        return call

    monkeypatch.setattr(runner, "_compiled_baseline", broken_compile)
    out = runner.run(cfg, device="cpu", warmup=1, budget_s=0.02)
    assert out.reference == "op_eager" and list(out.results) == ["op_eager", "custom"]
    assert out.skipped == {"op_compile": "RuntimeError: compile failed on purpose"}
    assert out.results["op_eager"].verified is None and out.results["op_eager"].speedup is None
    assert out.results["custom"].verified is True and out.results["custom"].speedup > 0
    path = save.save(cfg.name, cfg, out.results, "log\n", ref_label=out.reference, root=tmp_path, skipped=out.skipped)
    rec = json.loads(path.read_text())
    assert rec["skipped"] == out.skipped and set(rec["workloads"]) == {"op_eager", "custom"}
    table = view.rows(view.load(tmp_path))
    assert table[1][table[0].index("op_compile ms")] == "skip"
    assert "skipped" in runner.table(out)

    only = runner.run(cfg, device="cpu", warmup=1, budget_s=0.02, only=("custom",))
    assert list(only.results) == ["custom"] and only.results["custom"].verified is True


def test_op_compile_is_torch_compile_of_the_baseline():
    """The real op_compile entrant on the CPU (inductor's C++ backend): the compiled transformers experts
    forward equals op_eager bit for bit on a small shape."""
    cfg = _small_experts_config()
    cfg.custom = None
    out = runner.run(cfg, device="cpu", warmup=1, budget_s=0.02)
    assert out.skipped == {} and list(out.results) == ["op_eager", "op_compile"]
    assert out.results["op_compile"].verified is True


@pytest.mark.parametrize("layout", ["concat", "deepseek", "interleaved"])
def test_op_eager_baseline_is_the_transformers_forward(layout):
    """Each experts-level config's baseline builds the transformers experts module on the stand-in's
    tensors; on a small shape it equals the op_eager restatement (itself bit-exact against
    transformers' forward on the golden fixtures) bit for bit."""
    from cernels_amd.configs.registry import ExpertsConfig
    from cernels_amd.configs.synth import ACT_GPTOSS, LAYOUT_INTERLEAVED, ROUTER_TOPK_SOFTMAX, MoeShape
    from oracle import eager as O

    kw = dict(tokens=9, hidden=64, ffn=32, experts=8, top_k=2)
    if layout == "interleaved":
        kw.update(layout=LAYOUT_INTERLEAVED, act=ACT_GPTOSS, bias=True, router=ROUTER_TOPK_SOFTMAX)
    shape = MoeShape("deepseek_small" if layout == "deepseek" else f"{layout}_small", **kw)
    cfg = ExpertsConfig(shape)
    x, idx, w, m = cfg.inputs("cpu")
    with torch.no_grad():
        out = cfg.baseline(x, idx, w, m)
        again = cfg.baseline(x, idx, w, m)  # the module is built once per stand-in
    ref = O.experts_eager(x, idx, w, m.gate_up_proj, m.down_proj, m.gate_up_proj_bias, m.down_proj_bias,
                          layout=shape.layout, act=shape.act)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(out, again)


@pytest.mark.gpu
def test_reference_config_end_to_end(device, tmp_path):
    print("[benchmark runner] cohere2_moe_experts_decode", flush=True)
    out = runner.main("cohere2_moe_experts_decode", root=tmp_path, only=("op_eager", "custom"))
    results = out.results
    assert set(results) == {"op_eager", "custom"} and out.skipped == {}
    assert results["custom"].verified is True and results["custom"].speedup > 1.0
    rec = json.loads(next(tmp_path.glob("*/cohere2_moe_experts_decode.json")).read_text())
    assert rec["machine"]["gcn_arch"].startswith("gfx950")
