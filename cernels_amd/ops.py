"""Torch-facing MoE-experts ops over the C ABI (libcernels_moe.so).

Same names, argument order and error behaviour as the reference's torch ops
(src/kops/<slug>/torch-ext/torch_binding.cpp; C++ checks in csrc/<slug>.cu, e.g.
cohere2_moe_experts.cu:253-257 and :213-216): inputs must be contiguous CUDA tensors,
``x`` / expert weights bf16, ``indices`` int32, ``weights`` fp32 (gpt-oss biases fp32); a
violated contract raises ``RuntimeError``. Output is a new bf16 ``[T, H]`` tensor. Kernels run on
the current HIP stream of ``x``'s device, with no host synchronisation.

Scratch memory comes from torch's caching allocator and is handed to the library as a workspace.
"""

from __future__ import annotations

import ctypes

import torch

from cernels_amd import _native
from cernels_amd._native import (ACT_GELU_TANH, ACT_GPTOSS, ACT_RELU, ACT_SILU, ACT_SILU_PLAIN, LAYOUT_CONCAT,
                                 LAYOUT_INTERLEAVED, ROUTER_SOFTMAX_TOPK, ROUTER_TOPK_SOFTMAX, check)

# megablocks_moe's act_id (src/kops/registry/megablocks_moe.py:7 names them; csrc/megablocks_moe.cu:78-96)
# -> the library's non-gated activation
MEGABLOCKS_ACTS = {0: ACT_GELU_TANH, 1: ACT_SILU_PLAIN, 2: ACT_RELU}


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _check_inputs(x, gate_up_proj, down_proj, indices, weights, topk, layout, gate_up_bias=None, down_bias=None):
    tensors = [x, gate_up_proj, down_proj, indices, weights] + [t for t in (gate_up_bias, down_bias) if t is not None]
    _require(all(isinstance(t, torch.Tensor) for t in tensors), "inputs must be tensors")
    _require(all(t.is_cuda for t in tensors), "all inputs must be CUDA (HIP) tensors")
    _require(all(t.device == x.device for t in tensors), "all inputs must be on the same device")
    _require(all(t.is_contiguous() for t in tensors), "all inputs must be contiguous")
    _require(x.dtype == torch.bfloat16, "x must be bfloat16")
    _require(gate_up_proj.dtype == torch.bfloat16 and down_proj.dtype == torch.bfloat16, "expert weights must be bfloat16")
    _require(indices.dtype == torch.int32, "indices must be int32")
    _require(weights.dtype == torch.float32, "weights must be float32")
    _require(x.dim() == 2 and gate_up_proj.dim() == 3 and down_proj.dim() == 3, "x must be [T, H], weights [E, ., .]")
    T, H = x.shape
    E = gate_up_proj.size(0)
    if layout == LAYOUT_CONCAT:
        _require(gate_up_proj.size(2) == H and gate_up_proj.size(1) % 2 == 0, "gate_up_proj must be [E, 2F, H]")
        F = gate_up_proj.size(1) // 2
        _require(tuple(down_proj.shape) == (E, H, F), "down_proj must be [E, H, F]")
    else:
        _require(gate_up_proj.size(1) == H and gate_up_proj.size(2) % 2 == 0, "gate_up_proj must be [E, H, 2F]")
        F = gate_up_proj.size(2) // 2
        _require(tuple(down_proj.shape) == (E, F, H), "down_proj must be [E, F, H]")
    _require(tuple(indices.shape) == (T, int(topk)), "indices must be [T, topk]")
    _require(tuple(weights.shape) == (T, int(topk)), "weights must be [T, topk]")
    if gate_up_bias is not None:
        _require(gate_up_bias.dtype == torch.float32 and tuple(gate_up_bias.shape) == (E, 2 * F), "gate_up_bias must be fp32 [E, 2F]")
    if down_bias is not None:
        _require(down_bias.dtype == torch.float32 and tuple(down_bias.shape) == (E, H), "down_bias must be fp32 [E, H]")
    return int(T), int(H), int(F), int(E)


def moe_experts(
    x: torch.Tensor,
    gate_up_proj: torch.Tensor,
    down_proj: torch.Tensor,
    indices: torch.Tensor,
    weights: torch.Tensor,
    topk: int,
    *,
    layout: int = LAYOUT_CONCAT,
    act: int = ACT_SILU,
    gate_up_bias: torch.Tensor | None = None,
    down_bias: torch.Tensor | None = None,
    decode: bool = False,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Routed experts forward through the native library (prefill grouped GEMM or decode GEMV)."""
    T, H, F, E = _check_inputs(x, gate_up_proj, down_proj, indices, weights, topk, layout, gate_up_bias, down_bias)
    K = int(topk)
    L = _native.lib()
    if out is None:
        out = torch.empty((T, H), dtype=torch.bfloat16, device=x.device)
    else:
        _require(isinstance(out, torch.Tensor) and out.is_cuda and out.device == x.device and out.is_contiguous()
                 and out.dtype == torch.bfloat16 and tuple(out.shape) == (T, H),
                 "out must be a contiguous bf16 CUDA tensor [T, H] on x's device")
    if T == 0:
        return out
    with torch.cuda.device(x.device):
        if decode:
            nbytes = L.cernels_moe_experts_decode_workspace_bytes(T, H, F, E, K)
            fn, name = L.cernels_moe_experts_decode, "cernels_moe_experts_decode"
        else:
            nbytes = L.cernels_moe_experts_workspace_bytes(T, H, F, E, K)
            fn, name = L.cernels_moe_experts, "cernels_moe_experts"
        _require(nbytes > 0, f"{name}: invalid dimensions T={T} H={H} F={F} E={E} K={K}")
        ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        st = fn(
            _ptr(x), _ptr(gate_up_proj), _ptr(gate_up_bias), _ptr(down_proj), _ptr(down_bias), _ptr(indices),
            _ptr(weights), T, H, F, E, K, layout, act, _ptr(out), _ptr(ws), ctypes.c_size_t(nbytes),
            _stream(x.device),
        )
        check(st, name)
    return out


class PackedExperts:
    """Expert weights re-laid once in MFMA-fragment order for the packed prefill entry.

    ``gate_up`` / ``down`` hold the packed projections (uint8 buffers from ``pack_weights``: bf16
    fragments, fp16 fragments plus a power-of-two table for the down projection); biases are kept
    fp32 in their original column order (``bias_layout``).
    """

    def __init__(self, gate_up, down, H, F, E, act, bias_layout, gate_up_bias=None, down_bias=None):
        self.gate_up, self.down = gate_up, down
        self.H, self.F, self.E = int(H), int(F), int(E)
        self.act, self.bias_layout = act, bias_layout
        self.gate_up_bias, self.down_bias = gate_up_bias, down_bias


def pack_weights(weight: torch.Tensor, layout: int, which: int, H: int, F: int,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """One projection of every expert, packed by cernels_moe_pack_weights (runs on weight's stream).

    The result is a uint8 buffer of ``cernels_moe_packed_weight_bytes`` bytes: the source's element
    count for the first projections (bf16), and for DOWN the fp16 fragments followed by a table of one
    power of two per expert and 32-column fragment.
    """
    _require(weight.is_cuda and weight.dtype == torch.bfloat16 and weight.is_contiguous() and weight.dim() == 3,
             "weight must be a contiguous bf16 CUDA tensor [E, ., .]")
    E = int(weight.size(0))
    L = _native.lib()
    nbytes = L.cernels_moe_packed_weight_bytes(H, F, E, which)
    _require(nbytes >= weight.numel() * 2, f"cannot pack H={H} F={F} (need H % 64 == 0, F % 64 == 0)")
    if out is None:
        out = torch.empty(nbytes, dtype=torch.uint8, device=weight.device)
    _require(out.dtype == torch.uint8 and out.is_contiguous() and out.numel() == nbytes
             and out.device == weight.device, "out must be a contiguous uint8 buffer of the packed size")
    with torch.cuda.device(weight.device):
        st = L.cernels_moe_pack_weights(_ptr(weight), H, F, E, layout, which, _ptr(out), _stream(weight.device))
    check(st, "cernels_moe_pack_weights")
    return out


def split_shared_expert(shared_gate, shared_up, shared_down, F: int):
    """A dense SwiGLU MLP (gate/up [F_s, H], down [H, F_s]) as S = ceil(F_s/F) experts of width F in
    the concat layout: (gate_up [S, 2F, H], down [S, H, F]). Block i holds intermediate columns
    iF..iF+F-1; the last block is zero-padded, which adds silu(0)·0 = 0. Summing the S experts'
    outputs gives the MLP's output."""
    Fs, H = map(int, shared_gate.shape)
    _require(tuple(shared_up.shape) == (Fs, H) and tuple(shared_down.shape) == (H, Fs), "shared expert shapes")
    S = -(-Fs // F)
    pad = S * F - Fs
    g = torch.nn.functional.pad(shared_gate, (0, 0, 0, pad)).reshape(S, F, H)
    u = torch.nn.functional.pad(shared_up, (0, 0, 0, pad)).reshape(S, F, H)
    gu = torch.cat([g, u], dim=1).contiguous()
    dn = torch.nn.functional.pad(shared_down, (0, pad)).reshape(H, S, F).permute(1, 0, 2).contiguous()
    return gu, dn


def pack_experts_with_shared(gate_up_proj, down_proj, shared_gate, shared_up, shared_down) -> tuple[PackedExperts, int]:
    """Routed experts (concat layout, no biases) plus a dense SwiGLU shared expert, packed as one set.

    The shared expert ``down(silu(gate x) * up x)`` with intermediate size F_s becomes S = ceil(F_s/F)
    experts E..E+S-1 of width F: its gate/up rows and down columns are cut into S blocks, the last
    zero-padded (silu(0)·0 = 0, so padding adds nothing). The sum over the S blocks is the shared
    expert's output, so routing every token to E..E+S-1 with weight sigmoid(x·g) adds the gated
    shared expert (modeling_qwen3_next.py:789-795). Returns (packed, S).
    """
    E, F2, H = map(int, gate_up_proj.shape)
    F = F2 // 2
    sgu, sdn = split_shared_expert(shared_gate, shared_up, shared_down, F)
    S = int(sgu.shape[0])
    gu = pack_weights(torch.cat([gate_up_proj, sgu], dim=0).contiguous(), LAYOUT_CONCAT, _native.GATE_UP, H, F)
    dn = pack_weights(torch.cat([down_proj, sdn], dim=0).contiguous(), LAYOUT_CONCAT, _native.DOWN, H, F)
    return PackedExperts(gu, dn, H, F, E + S, ACT_SILU, LAYOUT_CONCAT), S


def pack_experts(gate_up_proj, down_proj, *, layout=LAYOUT_CONCAT, act=ACT_SILU, gate_up_bias=None,
                 down_bias=None) -> PackedExperts:
    """Pack both projections (either source layout) for moe_experts_packed."""
    E = int(gate_up_proj.size(0))
    if layout == LAYOUT_CONCAT:
        F, H = int(gate_up_proj.size(1)) // 2, int(gate_up_proj.size(2))
    else:
        H, F = int(gate_up_proj.size(1)), int(gate_up_proj.size(2)) // 2
    gu = pack_weights(gate_up_proj, layout, _native.GATE_UP, H, F)
    dn = pack_weights(down_proj, layout, _native.DOWN, H, F)
    f32 = lambda t: None if t is None else t.float().contiguous()  # noqa: E731
    return PackedExperts(gu, dn, H, F, E, act, layout, f32(gate_up_bias), f32(down_bias))


def moe_experts_packed(x: torch.Tensor, packed: PackedExperts, indices: torch.Tensor, weights: torch.Tensor,
                       topk: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """Routed experts prefill on packed weights (same result contract as moe_experts)."""
    _require(isinstance(packed, PackedExperts), "packed must come from pack_experts")
    _require(isinstance(x, torch.Tensor) and x.is_cuda and x.dtype == torch.bfloat16 and x.is_contiguous()
             and x.dim() == 2, "x must be a contiguous bf16 CUDA tensor [T, H]")
    dev = x.device
    for t, name in ((indices, "indices"), (weights, "weights"), (packed.gate_up, "packed gate_up"),
                    (packed.down, "packed down"), (packed.gate_up_bias, "gate_up_bias"),
                    (packed.down_bias, "down_bias")):
        if t is None and name.endswith("bias"):
            continue
        _require(isinstance(t, torch.Tensor) and t.is_cuda and t.device == dev and t.is_contiguous(),
                 f"{name} must be a contiguous CUDA tensor on x's device ({dev})")
    _require(indices.dtype == torch.int32, "indices must be int32")
    _require(weights.dtype == torch.float32, "weights must be float32")
    T, H = map(int, x.shape)
    K = int(topk)
    _require(H == packed.H and tuple(indices.shape) == (T, K) and tuple(weights.shape) == (T, K), "shape mismatch")
    for b, n in ((packed.gate_up_bias, 2 * packed.F), (packed.down_bias, packed.H)):
        _require(b is None or (b.dtype == torch.float32 and tuple(b.shape) == (packed.E, n)),
                 "biases must be float32 [E, 2F] and [E, H]")
    L = _native.lib()
    # the kernels read packed_weight_bytes(H, F, E) of each buffer: a buffer packed for other sizes is refused
    gu_which = _native.GATE_UP if packed.act in (ACT_SILU, ACT_GPTOSS) else _native.UP  # non-gated: w1 as UP
    for t, which, name in ((packed.gate_up, gu_which, "packed gate_up"), (packed.down, _native.DOWN, "packed down")):
        need = L.cernels_moe_packed_weight_bytes(packed.H, packed.F, packed.E, which)
        _require(need > 0 and t.dtype == torch.uint8 and t.numel() == need,
                 f"{name} must be the uint8 buffer pack_weights makes for H={packed.H} F={packed.F} E={packed.E}")
    if out is None:
        out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    else:
        _require(isinstance(out, torch.Tensor) and out.is_cuda and out.device == dev and out.is_contiguous()
                 and out.dtype == torch.bfloat16 and tuple(out.shape) == (T, H),
                 "out must be a contiguous bf16 CUDA tensor [T, H] on x's device")
    if T == 0:
        return out
    with torch.cuda.device(x.device):
        nbytes = L.cernels_moe_experts_workspace_bytes(T, H, packed.F, packed.E, K)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        st = L.cernels_moe_experts_packed(
            _ptr(x), _ptr(packed.gate_up), _ptr(packed.gate_up_bias), _ptr(packed.down), _ptr(packed.down_bias),
            _ptr(indices), _ptr(weights), T, H, packed.F, packed.E, K, packed.bias_layout, packed.act, _ptr(out),
            _ptr(ws), ctypes.c_size_t(nbytes), _stream(x.device))
    check(st, "cernels_moe_experts_packed")
    return out


def moe_router(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, top_k: int, mode: int,
               renorm: bool = True, want_logits: bool = False, shared_slots: int = 0):
    """Fused router: (indices [T,K+S] int32, weights [T,K+S] float32[, logits [T,E'] bf16]).

    mode ROUTER_SOFTMAX_TOPK: softmax over bf16 logits in fp32, top-k, renormalised if ``renorm``
    (Qwen3NextTopKRouter); ROUTER_TOPK_SOFTMAX: top-k of the logits, softmax over the k values
    (GptOssTopKRouter). Weights are the bf16-rounded scores as float32; ties go to the lower id.
    ``shared_slots`` S > 0: the last row of ``weight`` is the shared-expert gate (E' = E + 1 rows);
    every token gets S more slots with ids E..E+S-1 and weight bf16(sigmoid(x · gate)).
    """
    _require(x.is_cuda and x.dtype == torch.bfloat16 and x.is_contiguous() and x.dim() == 2, "x must be bf16 [T, H]")
    _require(weight.device == x.device and weight.dtype == torch.bfloat16 and weight.is_contiguous()
             and weight.dim() == 2, "router weight must be bf16 [E, H] on x's device")
    T, H = map(int, x.shape)
    S = int(shared_slots)
    ER = int(weight.shape[0])
    E = ER - (1 if S > 0 else 0)
    K = int(top_k)
    _require(int(weight.shape[1]) == H and E >= 1, "router weight shape mismatch")
    if bias is not None:
        _require(bias.device == x.device and bias.dtype == torch.bfloat16 and bias.is_contiguous()
                 and tuple(bias.shape) == (ER,), "router bias must be bf16 [E'] on x's device")
    idx = torch.empty((T, K + S), dtype=torch.int32, device=x.device)
    wts = torch.empty((T, K + S), dtype=torch.float32, device=x.device)
    logits = torch.empty((T, ER), dtype=torch.bfloat16, device=x.device)
    if T > 0:
        L = _native.lib()
        with torch.cuda.device(x.device):
            st = L.cernels_moe_router(_ptr(x), _ptr(weight), _ptr(bias), T, H, E, K, int(mode), int(bool(renorm)), S,
                                      _ptr(idx), _ptr(wts), _ptr(logits), _stream(x.device))
        check(st, "cernels_moe_router")
    return (idx, wts, logits) if want_logits else (idx, wts)


def decode_supported(T: int, K: int, H: int, F: int, layout: int = LAYOUT_CONCAT) -> bool:
    """True if the decode entry accepts this shape (otherwise use the prefill entry)."""
    L = _native.lib()
    return (
        layout == LAYOUT_CONCAT
        and 1 <= T <= L.cernels_moe_decode_max_tokens()
        and T * K <= L.cernels_moe_decode_max_pairs()
        and H % 8 == 0 and F % 8 == 0 and H <= 4096 and F <= 4096
    )


def route(indices: torch.Tensor, num_experts: int, tile_m: int = 128):
    """Device routing only: (expert_offsets [E+1], sorted_pairs [T*K], tile_offsets [E+1],
    tile_expert [capacity], meta [2]) — the tensors the prefill GEMMs schedule from."""
    _require(indices.is_cuda and indices.dtype == torch.int32 and indices.is_contiguous() and indices.dim() == 2,
             "indices must be a contiguous int32 CUDA tensor [T, K]")
    T, K = map(int, indices.shape)
    L = _native.lib()
    cap = L.cernels_moe_route_tile_capacity(T, K, num_experts, tile_m)
    dev = indices.device
    i32 = dict(dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, **i32)
    pairs = torch.full((max(T * K, 1),), -1, **i32)
    toff = torch.empty(num_experts + 1, **i32)
    texp = torch.full((max(cap, 1),), -1, **i32)
    meta = torch.empty(2, **i32)
    nbytes = max(int(L.cernels_moe_route_workspace_bytes(T, K, num_experts)), 4)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        st = L.cernels_moe_route(_ptr(indices), T, K, num_experts, tile_m, _ptr(offsets), _ptr(pairs), _ptr(toff),
                                 _ptr(texp), _ptr(meta), _ptr(ws), ctypes.c_size_t(nbytes), _stream(dev))
    check(st, "cernels_moe_route")
    return offsets, pairs[: T * K], toff, texp, meta


# ---- the reference's per-model torch ops (same schemas) ---------------------------------------
#
# Prefill runs on packed weights: the first call with a given set of weight tensors packs them (one
# launch per projection) and keeps the packed copy for as long as gate_up_proj lives. The copy is used
# again only for the very same tensor objects (held as weak references and compared by identity) at
# the same storage pointer, in-place version counter and shape; a write through ``.data`` does not
# advance the counter: call ``forget_packed(gate_up_proj)`` after one. Memory: the packed copy holds
# as many bytes as the expert weights themselves (plus a table of one byte per 32 down columns), so
# while it is kept the experts occupy about twice their own size in HBM. Decode reads the weights as
# stored.

import weakref

# id(gate_up_proj) -> (weak references to the keyed tensors, key, PackedExperts); an entry goes when
# gate_up_proj is freed. (Tensors compare elementwise, so a WeakKeyDictionary cannot key on them;
# identity is what is meant.)
_PACKED: dict = {}


def _weak(t):
    return None if t is None else weakref.ref(t)


def _same_objects(refs, tensors) -> bool:
    return all((r is None and t is None) or (r is not None and t is not None and r() is t)
               for r, t in zip(refs, tensors))


def _packed_for(gate_up_proj, down_proj, layout, act, gate_up_bias=None, down_bias=None) -> PackedExperts:
    tensors = (gate_up_proj, down_proj, gate_up_bias, down_bias)
    key = tuple(None if t is None else (t.data_ptr(), t._version, tuple(t.shape)) for t in tensors) + (layout, act)
    hit = _PACKED.get(id(gate_up_proj))
    if hit is not None and _same_objects(hit[0], tensors) and hit[1] == key:
        return hit[2]
    with torch.no_grad():
        pk = pack_experts(gate_up_proj, down_proj, layout=layout, act=act, gate_up_bias=gate_up_bias,
                          down_bias=down_bias)
    tid = id(gate_up_proj)
    refs = (weakref.ref(gate_up_proj, lambda _r, tid=tid: _PACKED.pop(tid, None)),) + tuple(
        _weak(t) for t in tensors[1:])
    _PACKED[tid] = (refs, key, pk)
    return pk


def packed_copy(gate_up_proj) -> PackedExperts | None:
    """The packed copy kept for ``gate_up_proj``, if any."""
    hit = _PACKED.get(id(gate_up_proj))
    return hit[2] if hit is not None and hit[0][0]() is gate_up_proj else None


def forget_packed(gate_up_proj) -> None:
    """Drop the packed copy kept for ``gate_up_proj`` (after a write through ``.data``)."""
    if packed_copy(gate_up_proj) is not None:
        _PACKED.pop(id(gate_up_proj), None)


def _prefill_named(x, gate_up_proj, down_proj, indices, weights, topk, layout=LAYOUT_CONCAT, act=ACT_SILU,
                   gate_up_bias=None, down_bias=None):
    _check_inputs(x, gate_up_proj, down_proj, indices, weights, topk, layout, gate_up_bias, down_bias)
    if x.shape[0] == 0:
        return torch.empty((0, x.shape[1]), dtype=torch.bfloat16, device=x.device)
    pk = _packed_for(gate_up_proj, down_proj, layout, act, gate_up_bias, down_bias)
    return moe_experts_packed(x, pk, indices, weights, topk)


def cohere2_moe_experts(x, gate_up_proj, down_proj, indices, weights, topk):
    return _prefill_named(x, gate_up_proj, down_proj, indices, weights, topk)


def cohere2_moe_experts_decode(x, gate_up_proj, down_proj, indices, weights, topk):
    return moe_experts(x, gate_up_proj, down_proj, indices, weights, topk, decode=True)


def deepseek_ocr2_moe_experts(x, gate_up_proj, down_proj, indices, weights, topk):
    return _prefill_named(x, gate_up_proj, down_proj, indices, weights, topk)


def deepseek_ocr2_moe_experts_decode(x, gate_up_proj, down_proj, indices, weights, topk):
    return moe_experts(x, gate_up_proj, down_proj, indices, weights, topk, decode=True)


def qwen3_next_moe_experts(x, gate_up_proj, down_proj, indices, weights, topk):
    return _prefill_named(x, gate_up_proj, down_proj, indices, weights, topk)


def gpt_oss_moe_experts(x, gate_up_proj, gate_up_bias, down_proj, down_bias, indices, weights, topk):
    return _prefill_named(x, gate_up_proj, down_proj, indices, weights, topk, layout=LAYOUT_INTERLEAVED,
                          act=ACT_GPTOSS, gate_up_bias=gate_up_bias, down_bias=down_bias)


def pack_experts_nongated(w1: torch.Tensor, w2: torch.Tensor, act: int) -> PackedExperts:
    """Pack megablocks-layout experts (w1 [E, H, F], w2 [E, F, H]) for moe_experts_packed with a
    non-gated activation (ACT_GELU_TANH, ACT_SILU_PLAIN or ACT_RELU)."""
    _require(act in MEGABLOCKS_ACTS.values(), "act must be a non-gated activation")
    _require(w1.dim() == 3 and w2.dim() == 3, "w1 [E, H, F] and w2 [E, F, H]")
    E, H, F = map(int, w1.shape)
    _require(tuple(w2.shape) == (E, F, H), "w2 must be [E, F, H]")
    up = pack_weights(w1.contiguous(), LAYOUT_INTERLEAVED, _native.UP, H, F)
    dn = pack_weights(w2.contiguous(), LAYOUT_INTERLEAVED, _native.DOWN, H, F)
    return PackedExperts(up, dn, H, F, E, act, LAYOUT_CONCAT)


def megablocks_moe(x, w1, w2, indices, weights, topk, act_id):
    """megablocks_moe(x [T,H], w1 [E,H,F], w2 [E,F,H], indices [T,topk] int32, weights [T,topk] fp32,
    topk, act_id) -> [T,H] bf16 (src/kops/megablocks_moe/torch-ext/torch_binding.cpp,
    csrc/megablocks_moe.cu:141-254): sum_k weights * act(x w1[e]) w2[e], act_id 0 = GELU (tanh form),
    1 = SiLU, 2 = ReLU. The weights are packed into the workspace on every call, as the op takes them
    as stored; the megablocks loader packs once per module instead."""
    _require(int(act_id) in MEGABLOCKS_ACTS, "act_id must be 0 (gelu), 1 (silu) or 2 (relu)")
    for t, name in ((x, "x"), (w1, "w1"), (w2, "w2"), (indices, "indices"), (weights, "weights")):
        _require(t.is_cuda and t.is_contiguous(), f"{name} must be a contiguous CUDA tensor")
    _require(x.dtype == torch.bfloat16 and w1.dtype == torch.bfloat16 and w2.dtype == torch.bfloat16,
             "x, w1, w2 must be bf16")
    _require(indices.dtype == torch.int32 and weights.dtype == torch.float32, "indices int32, weights fp32")
    T, H = map(int, x.shape)
    E, H1, F = map(int, w1.shape)
    K = int(topk)
    _require(H1 == H and tuple(w2.shape) == (E, F, H), "w1 must be [E, H, F] and w2 [E, F, H]")
    _require(tuple(indices.shape) == (T, K) and tuple(weights.shape) == (T, K), "indices / weights must be [T, topk]")
    out = torch.empty((T, H), dtype=torch.bfloat16, device=x.device)
    if T == 0:
        return out
    L = _native.lib()
    with torch.cuda.device(x.device):
        nbytes = L.cernels_megablocks_moe_workspace_bytes(T, H, F, E, K)
        _require(nbytes > 0, f"unsupported shape H={H} F={F} (need H % 64 == 0, F % 64 == 0)")
        ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        st = L.cernels_megablocks_moe(_ptr(x), _ptr(w1), _ptr(w2), _ptr(indices), _ptr(weights), T, H, F, E, K,
                                      int(act_id), _ptr(out), _ptr(ws), ctypes.c_size_t(nbytes), _stream(x.device))
    check(st, "megablocks_moe")
    return out


__all__ = [
    "moe_experts", "route", "decode_supported", "PackedExperts", "pack_weights", "pack_experts", "moe_experts_packed",
    "cohere2_moe_experts", "cohere2_moe_experts_decode",
    "deepseek_ocr2_moe_experts", "deepseek_ocr2_moe_experts_decode",
    "qwen3_next_moe_experts", "gpt_oss_moe_experts", "megablocks_moe", "pack_experts_nongated", "moe_router",
    "split_shared_expert", "pack_experts_with_shared", "forget_packed", "packed_copy",
    "LAYOUT_CONCAT", "LAYOUT_INTERLEAVED", "ACT_SILU", "ACT_GPTOSS", "ACT_GELU_TANH", "ACT_SILU_PLAIN", "ACT_RELU",
]
