#!/usr/bin/env python3
"""Routed MoE-experts benchmark on one MI355X — prints ONE JSON line on stdout.

A step = one call of the experts op (route → gate_up GEMM+SwiGLU → down GEMM+weight → combine,
or the decode GEMV pair) over one batch of seeded synthetic input already resident in HBM,
through the C ABI with preallocated output and workspace. BASELINE.json's metric names no single
config, so the headline is the largest workload that fits one GPU: ``gpt_oss_20b_experts``
(T=4096, H=F=2880, E=32, top-4, 815 GFLOP per step). The other BASELINE
workloads are measured the same way and reported under ``per_config``.

Prefill runs on expert weights packed once in MFMA-fragment order (``cernels_moe_pack_weights``,
what the drop-in loaders cache on a module at first use); the pack itself is outside the timed
region and reported as ``pack_ms``. The same workload on the weights as stored (transformers
layout, ``cernels_moe_experts``) is timed beside it as ``native_layout``. Decode streams the
weights as stored.

For the gpt-oss and qwen3-next workloads, whose reference ops run the router inside the call, the
fused router (``cernels_moe_router``, seeded router weights) is timed on its own as well and
reported as ``router`` and ``op_ms_with_router``, beside the same router as torch ops (F.linear,
softmax, topk: what the reference's loaders run) as ``router.torch_ops_ms``. ``module_ops`` times the
reference's module-level configs ``gpt_oss_moe_experts``, ``qwen3_next_moe_experts`` and
``megablocks_moe`` through the drop-in loaders (router, and for qwen3 the gated shared expert, inside
the call).

Timing: W untimed warmup steps, then exactly K steps between two ``torch.cuda.synchronize()``;
the step time is the HIP-event time of the K steps / K, with no events between a step's kernels. A
second pass of K steps records HIP events between the kernels on the launch stream, which gives
each kernel's average duration (``stages``).
Cold cache: steps rotate over R copies of the expert weights so that the bytes touched per
rotation exceed 1 GiB (4x the 256 MB Infinity Cache).

``roofline`` describes the dominant kernel of the headline: algorithmic bytes (or FLOPs) of one
launch / its average duration, against MI355X's 8 TB/s HBM or 2.5 PFLOP/s dense bf16 MFMA peak,
whichever bounds that kernel at its arithmetic intensity. ``roofline.traffic`` is that kernel's
measured HBM bytes per launch: two child runs of this script under ``rocprofv3 --pmc FETCH_SIZE``
and ``--pmc WRITE_SIZE``, each counter scaled by what it reads for a 256 MiB device copy (started
before this process touches the GPU; skipped with --no-traffic). ``cpu_baseline`` times the
op_eager restatement (the reference's baseline) on the host CPU on the same inputs, for every
workload that ran (``per_config[...].cpu_baseline``; the headline's is the top-level one).
``calibration`` times torch's own dense bf16 GEMM (hipBLASLt) on the headline's per-expert shapes
and on a large square GEMM: what the platform library reaches on this GPU, beside the peak.
"""

from __future__ import annotations

import argparse
import csv
import ctypes
import json
import math
import os
import shutil
import statistics
import subprocess
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFS = 2500.0
RIDGE = MFMA_BF16_PEAK_TFS * 1e12 / (HBM_PEAK_GBS * 1e9)  # FLOP/byte
METRIC = "MoE experts prefill TFLOP/s + decode HBM GB/s (% roofline), 1 MI355X"
COLD_BYTES = 1 << 30
CAL_MIB = 256
# kernel-name fragments of each stage's kernels in a rocprofv3 trace
# workloads whose reference op call runs the router inside it (src/kops/registry/gpt_oss_moe_experts.py:35,
# src/kops/registry/qwen3_next_moe_experts.py:28): the fused router is timed beside the experts op
ROUTER_IN_OP = {"gpt_oss_20b_experts": ("topk_softmax", True), "qwen3_next_zipf": ("softmax_topk", False)}
KERNEL_OF_STAGE = {
    "packed": {"gate_up": "moe_gemm_packed_kernel<0", "down": "moe_gemm_packed_kernel<1"},
    "native": {"gate_up": "moe_gemm_v3_kernel<0", "down": "moe_gemm_v3_kernel<1"},
}


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


def stage_model(shape, U, P, stage, path="packed"):
    """Algorithmic FLOPs and HBM bytes of one launch of a stage (each distinct expert once).

    Y (the down GEMM's per-pair rows, read back by the combine) is 24-bit floats (3 bytes) on the packed
    path and fp32 on the stored-layout path; glu is fp16 (packed) or bf16, 2 bytes either way (the packed
    path's exponent byte per 16 glu columns, P*F/16 bytes, is an implementation cost and not counted). The
    gpt-oss down bias is counted with the down stage although the packed path's combine reads it."""
    T, H, F, E = shape.tokens, shape.hidden, shape.ffn, shape.experts
    if stage == "route":
        return 0.0, P * 4 * 2 + (E + 1) * 8
    if stage == "gate_up":  # weights + fp32 bias, x read, glu bf16 written, pair ids + weights
        w = U * 2 * F * H * 2 + (U * 2 * F * 4 if shape.bias else 0)
        return 2.0 * P * H * 2 * F, w + T * H * 2 + P * F * 2 + P * 8
    y_bytes = P * H * 3 if path == "packed" else P * H * 4
    if stage == "down":  # weights + fp32 bias, glu read, weighted rows Y written
        w = U * H * F * 2 + (U * H * 4 if shape.bias else 0)
        return 2.0 * P * F * H, w + P * F * 2 + y_bytes + P * 8
    if stage == "combine":
        return float(P * H), y_bytes + T * H * 2 + P * 4
    if stage == "decode_gate_up":
        return 2.0 * P * H * 2 * F, U * 2 * F * H * 2 + T * H * 2 + P * F * 2
    if stage == "decode_down":
        return 2.0 * P * F * H, U * H * F * 2 + P * F * 2 + T * H * 2
    if stage == "router":  # x and the router weight (+ bias) read once, ids + fp32 weights written
        return 2.0 * T * H * E, T * H * 2 + E * H * 2 + (E * 2 if shape.bias else 0) + P * 8
    raise KeyError(stage)


def roofline_of(flops, nbytes, ms):
    ai = flops / nbytes if nbytes else 0.0
    if ai >= RIDGE:
        ach = flops / (ms * 1e-3) / 1e12
        return dict(bound="mfma", achieved=ach, peak=MFMA_BF16_PEAK_TFS, unit="TFLOP/s", frac=ach / MFMA_BF16_PEAK_TFS,
                    intensity=ai)
    ach = nbytes / (ms * 1e-3) / 1e9
    return dict(bound="hbm", achieved=ach, peak=HBM_PEAK_GBS, unit="GB/s", frac=ach / HBM_PEAK_GBS, intensity=ai)


def _timed_steps(step, stages, steps, warmup, hip, stream):
    """Runs warmup + timed steps; returns (ms per step, wall ms per step, {stage: mean ms}).

    The step time comes from K steps with no events between their kernels (only the two events
    around the K steps). A second pass of K steps records an event between every two kernels for
    the per-stage breakdown; those events add a little time of their own, so the stage times sum to
    slightly more than the step time."""
    import torch

    for i in range(warmup):
        step(i, None)
    torch.cuda.synchronize()
    nst = len(stages) + 1
    ev = Events(hip, nst * steps + 2)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    hip.hipEventRecord(ev.ev[0], ctypes.c_void_p(stream))
    for s in range(steps):
        step(s, None)
    hip.hipEventRecord(ev.ev[1], ctypes.c_void_p(stream))
    torch.cuda.synchronize()
    wall = (time.perf_counter() - wall0) * 1e3 / steps
    ms = ev.ms(0, 1) / steps
    stage_ms = {}
    if stages:
        arrs_keep = [(ctypes.c_void_p * nst)(*ev.ev[2 + s * nst: 2 + (s + 1) * nst]) for s in range(steps)]
        arrs = [ctypes.cast(a, ctypes.c_void_p) for a in arrs_keep]
        for s in range(steps):
            step(s, arrs[s])
        torch.cuda.synchronize()
        stage_ms = {name: statistics.mean(ev.ms(2 + s * nst + j, 2 + s * nst + j + 1) for s in range(steps))
                    for j, name in enumerate(stages)}
    ev.close()
    return ms, wall, stage_ms


def _torch_router_ms(kind, x, w, b, k, steps, warmup):
    """The reference's router as its transformers module computes it, in torch ops on the GPU
    (GptOssTopKRouter modeling_gpt_oss.py:126-130, Qwen3NextTopKRouter modeling_qwen3_next.py:766-775)."""
    import torch
    import torch.nn.functional as F

    def run():
        logits = F.linear(x, w, b)
        if kind == "topk_softmax":
            v, i = torch.topk(logits, k, dim=-1)
            return torch.softmax(v, dim=1, dtype=v.dtype), i
        p = torch.softmax(logits, dtype=torch.float, dim=-1)
        v, i = torch.topk(p, k, dim=-1)
        return (v / v.sum(dim=-1, keepdim=True)).to(logits.dtype), i

    for _ in range(warmup):
        run()
    a, z = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    for _ in range(steps):
        run()
    z.record()
    torch.cuda.synchronize()
    return a.elapsed_time(z) / steps


def run_config(shape, steps, warmup, dev, hip, log, with_native=True):
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
    stream = torch.cuda.current_stream(dev).cuda_stream
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    paths = {}

    if shape.decode:
        nbytes = L.cernels_moe_experts_decode_workspace_bytes(T, H, F, E, K)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)

        def step(i, ev_arr):
            st = L.cernels_moe_experts_decode_staged(ptr(x), ptr(W1[i % copies]), ptr(b1), ptr(W2[i % copies]),
                                                     ptr(b2), ptr(idx), ptr(rw), T, H, F, E, K, layout, act, ptr(out),
                                                     ptr(ws), ctypes.c_size_t(nbytes), stream, ev_arr)
            _native.check(st, shape.name)

        paths["decode"] = _timed_steps(step, ["decode_gate_up", "decode_down"], steps, warmup, hip, stream)
        main_path = "decode"
        pack_ms = None
    else:
        nbytes = L.cernels_moe_experts_workspace_bytes(T, H, F, E, K)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        stages = ["route", "gate_up", "down", "combine"]
        # one-time packing of every weight copy (timed on its own, outside the steps)
        pk = []
        ev = Events(hip, 2)
        hip.hipEventRecord(ev.ev[0], ctypes.c_void_p(stream))
        for c in range(copies):
            p1 = torch.empty(L.cernels_moe_packed_weight_bytes(H, F, E, _native.GATE_UP), dtype=torch.uint8, device=dev)
            p2 = torch.empty(L.cernels_moe_packed_weight_bytes(H, F, E, _native.DOWN), dtype=torch.uint8, device=dev)
            _native.check(L.cernels_moe_pack_weights(ptr(W1[c]), H, F, E, layout, _native.GATE_UP, ptr(p1), stream),
                          "pack gate_up")
            _native.check(L.cernels_moe_pack_weights(ptr(W2[c]), H, F, E, layout, _native.DOWN, ptr(p2), stream),
                          "pack down")
            pk.append((p1, p2))
        hip.hipEventRecord(ev.ev[1], ctypes.c_void_p(stream))
        torch.cuda.synchronize()
        pack_ms = ev.ms(0, 1) / copies
        ev.close()

        def step_packed(i, ev_arr):
            p1, p2 = pk[i % copies]
            st = L.cernels_moe_experts_packed_staged(ptr(x), ptr(p1), ptr(b1), ptr(p2), ptr(b2), ptr(idx), ptr(rw), T, H,
                                                     F, E, K, layout, act, ptr(out), ptr(ws), ctypes.c_size_t(nbytes),
                                                     stream, ev_arr)
            _native.check(st, shape.name)

        paths["packed"] = _timed_steps(step_packed, stages, steps, warmup, hip, stream)
        main_path = "packed"
        del pk
        if with_native:
            def step_native(i, ev_arr):
                st = L.cernels_moe_experts_staged(ptr(x), ptr(W1[i % copies]), ptr(b1), ptr(W2[i % copies]), ptr(b2),
                                                  ptr(idx), ptr(rw), T, H, F, E, K, layout, act, ptr(out), ptr(ws),
                                                  ctypes.c_size_t(nbytes), stream, ev_arr)
                _native.check(st, shape.name)

            paths["native"] = _timed_steps(step_native, stages, steps, warmup, hip, stream)

    router = None
    if shape.name in ROUTER_IN_OP:
        kind, with_bias = ROUTER_IN_OP[shape.name]
        g = torch.Generator().manual_seed(7)
        rw_w = (torch.randn(E, H, generator=g) * 0.02).bfloat16().to(dev)
        rw_b = (torch.randn(E, generator=g) * 0.02).bfloat16().to(dev) if with_bias else None
        r_idx = torch.empty((T, K), dtype=torch.int32, device=dev)
        r_wt = torch.empty((T, K), dtype=torch.float32, device=dev)
        r_lg = torch.empty((T, E), dtype=torch.bfloat16, device=dev)
        mode = _native.ROUTER_TOPK_SOFTMAX if kind == "topk_softmax" else _native.ROUTER_SOFTMAX_TOPK

        def step_router(i, ev_arr):
            _native.check(L.cernels_moe_router(ptr(x), ptr(rw_w), ptr(rw_b), T, H, E, K, mode, 1, 0, ptr(r_idx),
                                               ptr(r_wt), ptr(r_lg), stream), "router")

        rms, _, _ = _timed_steps(step_router, [], steps, warmup, hip, stream)
        router = dict(ms=rms, mode=kind, **roofline_of(*stage_model(shape, U, P, "router"), rms))
        router["torch_ms"] = _torch_router_ms(kind, x, rw_w, rw_b, K, steps, warmup)
        del rw_w, rw_b, r_idx, r_wt, r_lg

    ms, wall, stage_ms = paths[main_path]
    flops = shape.flops()
    alg_bytes = touched + 2 * T * H * 2 + P * 8
    t_roof_ms = max(flops / (MFMA_BF16_PEAK_TFS * 1e12), alg_bytes / (HBM_PEAK_GBS * 1e9)) * 1e3
    rec = dict(
        workload=shape.name, decode=shape.decode, path=main_path, tokens=T, hidden=H, ffn=F, experts=E, top_k=K,
        distinct_experts=U, weight_copies=copies, ms=ms, wall_ms_per_step=wall,
        tflops=flops / (ms * 1e-3) / 1e12, gbs=alg_bytes / (ms * 1e-3) / 1e9,
        mfma_peak_frac=flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFS,
        hbm_peak_frac=alg_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        attainable_frac=t_roof_ms / ms, algorithmic_bytes=alg_bytes, flops=flops,
        stages={k: dict(ms=v, **roofline_of(*stage_model(shape, U, P, k, main_path), v)) for k, v in stage_ms.items()},
    )
    if pack_ms is not None:
        rec["pack_ms"] = pack_ms
    if router is not None:
        rec["router"] = router
        rec["op_ms_with_router"] = ms + router["ms"]
    if "native" in paths:
        nms, _, nst = paths["native"]
        rec["native_layout"] = dict(ms=nms, tflops=flops / (nms * 1e-3) / 1e12, stages_ms=nst)
    log(f"[{shape.name}] {main_path}: {ms:.4f} ms/step  {rec['tflops']:.1f} TFLOP/s  {rec['gbs']:.0f} GB/s  "
        f"attainable {rec['attainable_frac'] * 100:.1f}%  stages " +
        " ".join(f"{k}={v['ms'] * 1e3:.1f}us" for k, v in rec["stages"].items()) +
        (f"  | native layout {rec['native_layout']['ms'] * 1e3:.1f}us" if "native_layout" in rec else "") +
        (f"  | pack {pack_ms:.2f} ms once" if pack_ms is not None else "") +
        (f"  | router {router['ms'] * 1e3:.1f}us ({router['frac'] * 100:.1f}% of {router['bound']} peak; "
         f"torch ops {router['torch_ms'] * 1e3:.1f}us)"
         if router is not None else ""))
    del W1, W2, ws, out
    torch.cuda.empty_cache()
    return rec


MODULE_OPS = ("gpt_oss_moe_experts", "qwen3_next_moe_experts", "megablocks_moe")


def run_module_op(name, steps, warmup, dev, log):
    """The reference's module-level op as its config calls it (src/configs/registry/{gpt_oss,qwen3_next}_moe_experts.py,
    megablocks_moe.py):
    the drop-in loader ``kernel(x, mlp)`` / ``kernel(x, block)`` with the router (and for qwen3 the gated
    shared expert) inside the call, Python dispatch included, on seeded weights and near-uniform routing
    as the reference's configs have it. Packing happens in the first warmup call."""
    import torch

    from cernels_amd.configs.registry import CONFIGS

    cfg = CONFIGS[name]
    t0 = time.time()
    x, mod = cfg.inputs(dev)
    log(f"[{name}] module inputs built in {time.time() - t0:.1f}s")
    s = cfg.shape
    T, H, F, E, K = s.tokens, s.hidden, s.ffn, s.experts, s.top_k
    flops = (6.0 if getattr(cfg, "gated", True) else 4.0) * T * K * H * F + 2.0 * T * H * E
    shared_f = 0
    if hasattr(mod, "shared_expert"):
        shared_f = int(mod.shared_expert.gate_proj.weight.shape[0])
        flops += 6.0 * T * H * shared_f + 2.0 * T * H
    for _ in range(max(1, warmup)):
        cfg.custom(x, mod)
    a, z = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    for _ in range(steps):
        cfg.custom(x, mod)
    z.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(z) / steps
    rec = dict(ms=ms, tflops=flops / (ms * 1e-3) / 1e12, tokens=T, hidden=H, ffn=F, experts=E, top_k=K,
               shared_ffn=shared_f, flops=flops)
    log(f"[{name}] module op (router{' + shared expert' if shared_f else ''} + experts): {ms:.4f} ms  "
        f"{rec['tflops']:.1f} TFLOP/s")
    del x, mod
    torch.cuda.empty_cache()
    return rec


def cpu_threads():
    """(threads used, CPUs in this process's affinity mask). The GPU boxes give each GPU a share of the
    host's cores and say so in OMP_NUM_THREADS; the baseline uses that whole share (or the whole
    affinity mask where no share is set)."""
    affinity = len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS") or 0)
    return (min(affinity, share) if share > 0 else affinity), affinity


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(shape, budget_s, log):
    """Times the op_eager restatement (oracle/eager.py, the reference's baseline path) on the host CPU
    on the workload's own inputs: one warmup run, then runs until ``budget_s`` is spent (at most 5)."""
    import torch

    from cernels_amd.configs.synth import make_inputs, make_weights
    from oracle import eager as O

    threads, affinity = cpu_threads()
    torch.set_num_threads(threads)
    inp, wts = make_inputs(shape), make_weights(shape)
    args = (inp.x, inp.top_k_index, inp.top_k_weights, wts.gate_up_proj, wts.down_proj, wts.gate_up_proj_bias,
            wts.down_proj_bias)
    kw = dict(layout=shape.layout, act=shape.act)
    t0 = time.perf_counter()
    O.experts_eager(*args, **kw)  # warmup
    warm = time.perf_counter() - t0
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 and (not times or time.perf_counter() - t_start + warm <= budget_s):
        t0 = time.perf_counter()
        O.experts_eager(*args, **kw)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    cpu = _cpu_model()
    flops = shape.flops()
    log(f"[cpu_baseline {shape.name}] {len(times)} runs, median {med * 1e3:.2f} ms on {threads} threads "
        f"({affinity} CPUs in the affinity mask; {cpu})")
    rec = dict(
        cores=torch.get_num_threads(), kind="port",
        sample=(f"op_eager restatement (transformers experts forward loop, oracle/eager.py) on the full "
                f"{shape.name} workload (T={shape.tokens}), bf16 on the host CPU, 1 warmup + {len(times)} timed "
                f"runs, median {med * 1e3:.2f} ms; {threads} threads = the GPU's share of the host "
                f"(OMP_NUM_THREADS; {affinity} CPUs in the affinity mask); CPU: {cpu}"),
        ms=med * 1e3, affinity_cpus=affinity,
    )
    if shape.decode:
        U = int(torch.unique(inp.top_k_index).numel())
        nbytes = U * shape.expert_bytes() + 2 * shape.tokens * shape.hidden * 2 + shape.pairs * 8
        rec.update(value=nbytes / med / 1e9, unit="GB/s")
    else:
        rec.update(value=flops / med / 1e12, unit="TFLOP/s")
    return rec


def dense_gemm_calibration(dev, log, reps=20):
    """torch's dense bf16 GEMM (hipBLASLt) on this GPU: the headline's per-expert GEMMs at the uniform
    load (T*k/E = 512 rows per expert) as one batched GEMM over its 32 experts, and an 8192^3 GEMM.
    Operands are contiguous (row-major A, row-major B)."""
    import torch

    res = {}
    shapes = {"gpt_oss_gate_up_bmm_32x512x2880x5760": (32, 512, 2880, 5760),
              "gpt_oss_down_bmm_32x512x2880x2880": (32, 512, 2880, 2880),
              "square_8192": (1, 8192, 8192, 8192)}
    for name, (b, m, k, n) in shapes.items():
        a = torch.randn(b, m, k, device=dev).bfloat16()
        w = torch.randn(b, k, n, device=dev).bfloat16()
        for _ in range(3):
            torch.bmm(a, w)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            torch.bmm(a, w)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        tf = 2.0 * b * m * k * n / (ms * 1e-3) / 1e12
        res[name] = dict(ms=round(ms, 5), tflops=round(tf, 1), mfma_peak_frac=round(tf / MFMA_BF16_PEAK_TFS, 4))
        log(f"[calibration] torch.bmm bf16 {name}: {ms:.4f} ms, {tf:.1f} TFLOP/s ({tf / MFMA_BF16_PEAK_TFS * 100:.1f}% "
            f"of the {MFMA_BF16_PEAK_TFS:.0f} TFLOP/s peak)")
        del a, w
    torch.cuda.empty_cache()
    return res


# ---- the reference's benchmark runner on its own config names -------------------------------------

REFERENCE_CONFIGS = ("cohere2_moe_experts", "cohere2_moe_experts_decode", "deepseek_ocr2_moe_experts",
                     "deepseek_ocr2_moe_experts_decode", "gpt_oss_moe_experts", "qwen3_next_moe_experts")


def run_reference_config(name, out_dir):
    """One config through cernels_amd.benchmark (the reference's src/benchmark/main.py protocol: op_eager =
    the transformers module, custom = the drop-in loader, verify, blocked_autorange), its record saved
    under ``out_dir``; returns the record's workloads."""
    from dataclasses import asdict

    from cernels_amd.benchmark import main as runner

    outcome = runner.main(name, root=out_dir)
    rec = {w: asdict(r) for w, r in outcome.results.items()}
    rec.update({w: {"skipped": why} for w, why in outcome.skipped.items()})
    return rec


# ---- HBM traffic per launch (rocprofv3 counters, child processes) ----------------------------------

def _inner_traffic(headline):
    """Child mode: a 256 MiB calibration copy, then a few packed steps of the headline workload."""
    import torch

    from cernels_amd.configs.registry import BASELINE_SHAPES

    dev = torch.device("cuda:0")
    n = CAL_MIB << 20
    src = torch.ones(n, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)  # the first copyBuffer dispatch of this process: the calibration copy
    torch.cuda.synchronize()
    del src, dst
    run_config(BASELINE_SHAPES[headline], 5, 2, dev, _hip(), lambda m: None, with_native=False)


def _counter_rows(path):
    with open(path) as f:
        return list(csv.DictReader(f))


def measure_traffic(headline, log, timeout_s=180):
    """Per-launch HBM MB of the headline's packed kernels from FETCH_SIZE / WRITE_SIZE passes."""
    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(prof):
        return None, "rocprofv3 not found"
    res = {}
    with tempfile.TemporaryDirectory(prefix="bench_pmc_") as tmp:
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            out = Path(tmp) / counter
            cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", str(out), "-o", "c", "--",
                   sys.executable, str(Path(__file__).resolve()), "--inner-traffic", headline]
            try:
                r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout_s, cwd=tmp,
                                   env=dict(os.environ, TMPDIR=tmp), start_new_session=True)
            except subprocess.TimeoutExpired:
                return None, f"rocprofv3 --pmc {counter} timed out"
            files = list(out.rglob("*counter_collection.csv"))
            if not files:
                return None, f"rocprofv3 --pmc {counter} wrote no counters (rc={r.returncode})"
            rows = _counter_rows(files[0])
            rows.sort(key=lambda r: int(r["Dispatch_Id"]))
            cal = next((float(r["Counter_Value"]) for r in rows if "copyBuffer" in r["Kernel_Name"]), None)
            if not cal:
                return None, "calibration copy not found in the trace"
            scale = (CAL_MIB * 1024) / cal  # true KiB per counted KiB
            per = {}
            for stage, frag in KERNEL_OF_STAGE["packed"].items():
                vals = [float(r["Counter_Value"]) for r in rows if frag in r["Kernel_Name"]]
                if vals:
                    per[stage] = statistics.mean(vals) * scale * 1024 / 1e6  # MB per launch
            res[counter] = dict(scale=scale, per_stage_mb=per)
    log(f"[traffic] FETCH scale {res['FETCH_SIZE']['scale']:.3f}, WRITE scale {res['WRITE_SIZE']['scale']:.3f}; "
        + ", ".join(f"{k} {res['FETCH_SIZE']['per_stage_mb'].get(k, 0) + res['WRITE_SIZE']['per_stage_mb'].get(k, 0):.1f} MB"
                    for k in KERNEL_OF_STAGE["packed"]))
    return res, None


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--configs", default="all",
                    help="'all', 'headline', 'module' (only the module-level loader ops) or a comma list of BASELINE "
                         "workload names")
    ap.add_argument("--cpu-seconds", type=float, default=30.0,
                    help="CPU-baseline budget over all workloads that ran (split evenly; at least one run each)")
    ap.add_argument("--no-calibration", action="store_true", help="skip timing torch's dense GEMM")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-native", action="store_true", help="skip timing prefill on the weights as stored")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 FETCH/WRITE_SIZE child runs")
    ap.add_argument("--no-module-ops", action="store_true", help="skip the module-level gpt-oss / qwen3 loader timings")
    ap.add_argument("--reference-configs", metavar="NAMES",
                    help="run the reference's benchmark runner on its own config names (comma list or 'all'): "
                         "op_eager = the transformers module, custom = the drop-in loader; one JSON record each")
    ap.add_argument("--inner-traffic", metavar="WORKLOAD", help=argparse.SUPPRESS)
    ap.add_argument("--report", metavar="PATH", help="also write the full per-workload record (JSON) to PATH")
    ap.add_argument("--analysis-root", default="analysis",
                    help="--reference-configs: where the runner's <host>/<config>.{json,log} records go")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures the experts op on one GPU "
              "(collectives and sharding are design-only here); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.inner_traffic:
        _inner_traffic(args.inner_traffic)
        return

    from cernels_amd.configs.registry import BASELINE_ORDER, BASELINE_SHAPES, HEADLINE

    log = lambda m: print(m, file=sys.stderr, flush=True)  # noqa: E731
    traffic, traffic_note = (None, "skipped (--no-traffic)")
    if not args.no_traffic and not args.reference_configs:  # child processes first, before this process initialises the GPU
        traffic, traffic_note = measure_traffic(HEADLINE, log)

    import torch

    if not torch.cuda.is_available():
        log("bench.py: no GPU visible")
        sys.exit(1)
    dev = torch.device("cuda:0")
    hip = _hip()
    if args.reference_configs:
        names = REFERENCE_CONFIGS if args.reference_configs == "all" else args.reference_configs.split(",")
        recs = {n: run_reference_config(n, Path(args.analysis_root)) for n in names}
        print(json.dumps({"metric": "reference configs: custom vs op_eager (transformers module), ms per call",
                          "unit": "ms", "higher_is_better": False, "n_gpus": 1, "configs": recs}), flush=True)
        return
    if args.configs == "module":
        mods = {n: run_module_op(n, args.steps, args.warmup, dev, log) for n in MODULE_OPS}
        print(json.dumps({"metric": "module-level MoE ops (drop-in loaders), ms per call", "unit": "ms",
                          "higher_is_better": False, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                          "module_ops": {n: {k: (round(v, 5) if isinstance(v, float) else v) for k, v in r.items()}
                                         for n, r in mods.items()}}), flush=True)
        return
    if args.configs == "all":
        names = [HEADLINE] + [n for n in BASELINE_ORDER if n != HEADLINE]
    elif args.configs == "headline":
        names = [HEADLINE]
    else:
        names = [n.strip() for n in args.configs.split(",") if n.strip()]
    per = {}
    for n in names:
        per[n] = run_config(BASELINE_SHAPES[n], args.steps, args.warmup, dev, hip, log, with_native=not args.no_native)
    mods = {}
    if not args.no_module_ops and args.configs == "all":
        for n in MODULE_OPS:
            mods[n] = run_module_op(n, args.steps, args.warmup, dev, log)
    head = per.get(HEADLINE) or per[names[0]]
    dom_name, dom = max(head["stages"].items(), key=lambda kv: kv[1]["ms"])
    traffic_mb = None
    if traffic and head["path"] == "packed" and dom_name in traffic["FETCH_SIZE"]["per_stage_mb"]:
        traffic_mb = traffic["FETCH_SIZE"]["per_stage_mb"][dom_name] + traffic["WRITE_SIZE"]["per_stage_mb"].get(dom_name, 0.0)
    roofline = dict(bound=dom["bound"], achieved=round(dom["achieved"], 3), peak=dom["peak"], unit=dom["unit"],
                    frac=round(dom["frac"], 5),
                    traffic=None if traffic_mb is None else round(traffic_mb * 1e6),
                    traffic_unit="bytes per launch (HBM, rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated)",
                    kernel=dom_name, kernel_ms=round(dom["ms"], 5),
                    algorithmic_bytes=round(stage_model(BASELINE_SHAPES[head["workload"]], head["distinct_experts"],
                                                        BASELINE_SHAPES[head["workload"]].pairs, dom_name)[1]),
                    intensity_flop_per_byte=round(dom["intensity"], 2))
    if traffic_mb is None:
        roofline["traffic_note"] = traffic_note or "dominant kernel not in the counter trace"
    calibration = None if args.no_calibration else dense_gemm_calibration(dev, log)
    cpu = None
    if not args.no_cpu_baseline:
        for n in names:
            c = cpu_baseline(BASELINE_SHAPES[n], args.cpu_seconds / len(names), log)
            per[n]["cpu_baseline"] = {k: (round(v, 6) if isinstance(v, float) else v) for k, v in c.items()}
        cpu = per[head["workload"]]["cpu_baseline"]
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
        "data": "synthetic (seeded CPU-generated bf16 x ~ N(0,1), weights and biases ~ N(0,0.02), seeded router "
                "logits ~ N(0,1) routed as BASELINE.json states per config)",
        "config": {"workload": head["workload"], "tokens": head["tokens"], "hidden": head["hidden"],
                   "ffn": head["ffn"], "experts": head["experts"], "top_k": head["top_k"],
                   "weights": "packed once (MFMA-fragment order), pack time excluded" if head["path"] == "packed"
                   else "as stored",
                   "mfma_peak_frac": round(head["mfma_peak_frac"], 5),
                   "attainable_roofline_frac": round(head["attainable_frac"], 5)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "per_config": {
            n: {k: (round(v, 5) if isinstance(v, float) else v) for k, v in r.items()
                if k not in ("stages", "native_layout", "router", "cpu_baseline")}
            | {"stages_ms": {s: round(v["ms"], 5) for s, v in r["stages"].items()}}
            | ({"router": {"ms": round(r["router"]["ms"], 5), "mode": r["router"]["mode"], "bound": r["router"]["bound"],
                           "frac": round(r["router"]["frac"], 4), "torch_ops_ms": round(r["router"]["torch_ms"], 5)}}
               if "router" in r else {})
            | ({"native_layout_ms": round(r["native_layout"]["ms"], 5)} if "native_layout" in r else {})
            | ({"cpu_baseline": r["cpu_baseline"]} if "cpu_baseline" in r else {})
            for n, r in per.items()
        },
        "module_ops": {n: {k: (round(v, 5) if isinstance(v, float) else v) for k, v in r.items()} for n, r in mods.items()},
        "calibration": calibration,
    }
    if args.report:
        Path(args.report).parent.mkdir(parents=True, exist_ok=True)
        Path(args.report).write_text(json.dumps({"line": line, "per_config_full": per, "traffic": traffic}, indent=1,
                                                default=float))
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
