#!/usr/bin/env python3
"""Routed MoE-experts benchmark on one MI355X — prints ONE JSON line on stdout.

A step = one call of the experts op (route → gate_up GEMM+SwiGLU → down GEMM+weight → combine,
or the decode GEMV pair) over one batch of seeded synthetic input already resident in HBM,
through the C ABI with preallocated output and workspace. The headline is BASELINE.json
configs[1] (``deepseek_v2_lite_prefill``: T=2048, H=1280, F=896, E=64, top-6); the other
BASELINE workloads are measured the same way and reported under ``per_config``.

Timing: W untimed warmup steps, then exactly K steps between two ``torch.cuda.synchronize()``;
the step time is the HIP-event time of the K steps / K. Each step also records HIP events between
its kernels on the launch stream, which gives each kernel's average duration (``stages``).
Cold cache: steps rotate over R copies of the expert weights so that the bytes touched per
rotation exceed 1 GiB (4x the 256 MB Infinity Cache).

``roofline`` describes the dominant kernel of the headline: algorithmic bytes (or FLOPs) of one
launch / its average duration, against MI355X's 8 TB/s HBM or 2.5 PFLOP/s dense bf16 MFMA peak,
whichever bounds that kernel at its arithmetic intensity. ``cpu_baseline`` times the op_eager
restatement (the reference's baseline) on the host CPU on the same inputs.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFS = 2500.0
RIDGE = MFMA_BF16_PEAK_TFS * 1e12 / (HBM_PEAK_GBS * 1e9)  # FLOP/byte
METRIC = "MoE experts prefill TFLOP/s + decode HBM GB/s (% roofline), 1 MI355X"
COLD_BYTES = 1 << 30


def _hip():
    lib = ctypes.CDLL("libamdhip64.so.7")  # the runtime torch already loaded (same soname)
    lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
    return lib


class Events:
    def __init__(self, hip, n):
        self.hip, self.ev = hip, []
        for _ in range(n):
            e = ctypes.c_void_p()
            if hip.hipEventCreate(ctypes.byref(e)) != 0:
                raise RuntimeError("hipEventCreate failed")
            self.ev.append(e)

    def ms(self, a, b):
        out = ctypes.c_float()
        if self.hip.hipEventElapsedTime(ctypes.byref(out), self.ev[a], self.ev[b]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return out.value

    def close(self):
        for e in self.ev:
            self.hip.hipEventDestroy(e)


def stage_model(shape, U, P, stage):
    """Algorithmic FLOPs and HBM bytes of one launch of a stage (each distinct expert once)."""
    T, H, F, E = shape.tokens, shape.hidden, shape.ffn, shape.experts
    if stage == "route":
        return 0.0, P * 4 * 2 + (E + 1) * 8
    if stage == "gate_up":
        w = U * 2 * F * H * 2 + (U * 2 * F * 2 if shape.bias else 0)
        return 2.0 * P * H * 2 * F, w + T * H * 2 + P * F * 2 + P * 8
    if stage == "down":
        w = U * H * F * 2 + (U * H * 2 if shape.bias else 0)
        return 2.0 * P * F * H, w + P * F * 2 + P * H * 4 + P * 8
    if stage == "combine":
        return float(P * H), P * H * 4 + T * H * 2 + P * 4
    if stage == "decode_gate_up":
        return 2.0 * P * H * 2 * F, U * 2 * F * H * 2 + T * H * 2 + P * F * 2
    if stage == "decode_down":
        return 2.0 * P * F * H, U * H * F * 2 + P * F * 2 + T * H * 2
    raise KeyError(stage)


def roofline_of(flops, nbytes, ms):
    ai = flops / nbytes if nbytes else 0.0
    if ai >= RIDGE:
        ach = flops / (ms * 1e-3) / 1e12
        return dict(bound="mfma", achieved=ach, peak=MFMA_BF16_PEAK_TFS, unit="TFLOP/s", frac=ach / MFMA_BF16_PEAK_TFS,
                    intensity=ai)
    ach = nbytes / (ms * 1e-3) / 1e9
    return dict(bound="hbm", achieved=ach, peak=HBM_PEAK_GBS, unit="GB/s", frac=ach / HBM_PEAK_GBS, intensity=ai)


def run_config(shape, steps, warmup, dev, hip, log):
    import torch

    from cernels_amd import _native
    from cernels_amd.configs.synth import make_inputs, make_weights

    t0 = time.time()
    inp, wts = make_inputs(shape), make_weights(shape)
    log(f"[{shape.name}] inputs generated in {time.time() - t0:.1f}s")
    U = int(torch.unique(inp.top_k_index).numel())
    P = shape.pairs
    touched = U * shape.expert_bytes()
    copies = max(1, min(64, math.ceil(COLD_BYTES / max(touched, 1))))
    x = inp.x.to(dev)
    idx = inp.top_k_index.to(torch.int32).contiguous().to(dev)
    rw = inp.top_k_weights.float().contiguous().to(dev)
    W1 = [wts.gate_up_proj.to(dev)]
    W2 = [wts.down_proj.to(dev)]
    for _ in range(copies - 1):
        W1.append(W1[0].clone())
        W2.append(W2[0].clone())
    b1 = None if wts.gate_up_proj_bias is None else wts.gate_up_proj_bias.float().contiguous().to(dev)
    b2 = None if wts.down_proj_bias is None else wts.down_proj_bias.float().contiguous().to(dev)
    del wts
    L = _native.lib()
    T, H, F, E, K = shape.tokens, shape.hidden, shape.ffn, shape.experts, shape.top_k
    layout = _native.LAYOUT_INTERLEAVED if shape.layout == "interleaved" else _native.LAYOUT_CONCAT
    act = _native.ACT_GPTOSS if shape.act == "gptoss" else _native.ACT_SILU
    if shape.decode:
        nbytes = L.cernels_moe_experts_decode_workspace_bytes(T, H, F, E, K)
        fn, stages = L.cernels_moe_experts_decode_staged, ["decode_gate_up", "decode_down"]
    else:
        nbytes = L.cernels_moe_experts_workspace_bytes(T, H, F, E, K)
        fn, stages = L.cernels_moe_experts_staged, ["route", "gate_up", "down", "combine"]
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    nst = len(stages) + 1
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731

    def step(i, ev_arr):
        st = fn(ptr(x), ptr(W1[i % copies]), ptr(b1), ptr(W2[i % copies]), ptr(b2), ptr(idx), ptr(rw), T, H, F, E,
                K, layout, act, ptr(out), ptr(ws), ctypes.c_size_t(nbytes), stream, ev_arr)
        _native.check(st, shape.name)

    for i in range(warmup):
        step(i, None)
    torch.cuda.synchronize()
    ev = Events(hip, nst * steps + 2)
    arrs_keep = [(ctypes.c_void_p * nst)(*ev.ev[2 + s * nst: 2 + (s + 1) * nst]) for s in range(steps)]
    arrs = [ctypes.cast(a, ctypes.c_void_p) for a in arrs_keep]
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    hip.hipEventRecord(ev.ev[0], ctypes.c_void_p(stream))
    for s in range(steps):
        step(s, arrs[s])
    hip.hipEventRecord(ev.ev[1], ctypes.c_void_p(stream))
    torch.cuda.synchronize()
    wall = (time.perf_counter() - wall0) * 1e3 / steps
    ms = ev.ms(0, 1) / steps
    stage_ms = {}
    for j, name in enumerate(stages):
        vals = [ev.ms(2 + s * nst + j, 2 + s * nst + j + 1) for s in range(steps)]
        stage_ms[name] = statistics.mean(vals)
    ev.close()
    flops = shape.flops()
    alg_bytes = touched + 2 * T * H * 2 + P * 8
    t_roof_ms = max(flops / (MFMA_BF16_PEAK_TFS * 1e12), alg_bytes / (HBM_PEAK_GBS * 1e9)) * 1e3
    rec = dict(
        workload=shape.name, decode=shape.decode, tokens=T, hidden=H, ffn=F, experts=E, top_k=K,
        distinct_experts=U, weight_copies=copies, ms=ms, wall_ms_per_step=wall,
        tflops=flops / (ms * 1e-3) / 1e12, gbs=alg_bytes / (ms * 1e-3) / 1e9,
        mfma_peak_frac=flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFS,
        hbm_peak_frac=alg_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        attainable_frac=t_roof_ms / ms, algorithmic_bytes=alg_bytes, flops=flops,
        stages={k: dict(ms=v, **roofline_of(*stage_model(shape, U, P, k), v)) for k, v in stage_ms.items()},
    )
    log(f"[{shape.name}] {ms:.4f} ms/step  {rec['tflops']:.1f} TFLOP/s  {rec['gbs']:.0f} GB/s  "
        f"attainable {rec['attainable_frac'] * 100:.1f}%  stages " +
        " ".join(f"{k}={v['ms'] * 1e3:.1f}us" for k, v in rec["stages"].items()))
    del W1, W2, ws, out
    torch.cuda.empty_cache()
    return rec, (inp, shape)


def cpu_baseline(shape, budget_s, log):
    """Times the op_eager restatement on the host CPU on the headline workload's inputs."""
    import torch

    from cernels_amd.configs.synth import make_inputs, make_weights
    from oracle import eager as O

    cores = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(cores)
    inp, wts = make_inputs(shape), make_weights(shape)
    args = (inp.x, inp.top_k_index, inp.top_k_weights, wts.gate_up_proj, wts.down_proj)
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        O.experts_eager(*args)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s or len(times) >= 6:
            break
    timed = times[1:] if len(times) > 1 else times
    med = statistics.median(timed)
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    log(f"[cpu_baseline] {len(times)} runs, median {med * 1e3:.1f} ms on {cores} threads ({cpu})")
    return dict(
        value=shape.flops() / med / 1e12, unit="TFLOP/s", cores=torch.get_num_threads(), kind="port",
        sample=(f"op_eager restatement (transformers experts forward loop, oracle/eager.py) on the full "
                f"{shape.name} workload (T={shape.tokens}), bf16 on CPU, {len(times)} runs"
                f"{' after 1 warmup' if len(times) > 1 else ''}, median {med * 1e3:.1f} ms; CPU: {cpu}"),
        ms=med * 1e3,
    )


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--configs", default="all", help="'all', 'headline' or a comma list of BASELINE workload names")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--report", default=str(ROOT / "gpurun_out" / "bench_report.json"))
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="also run a plain device copy of this many MiB (a known-size kernel against which "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings are scaled)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures the experts op on one GPU "
              f"(the multi-GPU design is described in DESIGN.md); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    from cernels_amd.configs.registry import BASELINE_ORDER, BASELINE_SHAPES, HEADLINE

    log = lambda m: print(m, file=sys.stderr, flush=True)  # noqa: E731
    if not torch.cuda.is_available():
        log("bench.py: no GPU visible")
        sys.exit(1)
    dev = torch.device("cuda:0")
    hip = _hip()
    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[copy calibration] copied {args.copy_calibration_mib} MiB")
        del src, dst
    if args.configs == "all":
        names = [HEADLINE] + [n for n in BASELINE_ORDER if n != HEADLINE]
    elif args.configs == "headline":
        names = [HEADLINE]
    else:
        names = [n.strip() for n in args.configs.split(",") if n.strip()]
    per = {}
    for n in names:
        rec, _ = run_config(BASELINE_SHAPES[n], args.steps, args.warmup, dev, hip, log)
        per[n] = rec
    head = per.get(HEADLINE) or per[names[0]]
    dom_name, dom = max(head["stages"].items(), key=lambda kv: kv[1]["ms"])
    roofline = dict(bound=dom["bound"], achieved=round(dom["achieved"], 3), peak=dom["peak"], unit=dom["unit"],
                    frac=round(dom["frac"], 5), traffic=None, kernel=dom_name, kernel_ms=round(dom["ms"], 5),
                    intensity_flop_per_byte=round(dom["intensity"], 2))
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(BASELINE_SHAPES[head["workload"]], args.cpu_seconds, log)
        cpu = {k: (round(v, 6) if isinstance(v, float) else v) for k, v in cpu.items()}
    line = {
        "metric": METRIC,
        "value": round(head["tflops"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded CPU-generated bf16 x ~ N(0,1), weights ~ N(0,0.02), softmax top-k routing)",
        "config": {"workload": head["workload"], "tokens": head["tokens"], "hidden": head["hidden"],
                   "ffn": head["ffn"], "experts": head["experts"], "top_k": head["top_k"],
                   "mfma_peak_frac": round(head["mfma_peak_frac"], 5),
                   "attainable_roofline_frac": round(head["attainable_frac"], 5)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "per_config": {
            n: {k: (round(v, 5) if isinstance(v, float) else v) for k, v in r.items() if k != "stages"}
            | {"stages_ms": {s: round(v["ms"], 5) for s, v in r["stages"].items()}}
            for n, r in per.items()
        },
    }
    try:
        Path(args.report).parent.mkdir(parents=True, exist_ok=True)
        Path(args.report).write_text(json.dumps({"line": line, "per_config_full": per}, indent=1, default=float))
    except OSError:
        pass
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
