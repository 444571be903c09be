"""CPU oracle for the routed MoE-experts path — TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may import this
module; the product path (cernels_amd) never does.

What it restates (third-party algorithm: transformers 5.15.0, the reference pins >=5.10.2 in
pyproject.toml:15; the reference's configs call these modules as their op_eager baseline,
src/configs/registry/cohere2_moe_experts.py:81-85, gpt_oss_moe_experts.py:62-67):

* ``experts_eager``  — ``Cohere2MoeExperts.forward`` (models/cohere2_moe/modeling_cohere2_moe.py
  :114-138; DeepseekOcr2TextExperts :1150-1174 and Qwen3NextExperts :730-754 are the same code)
  and ``GptOssExperts.forward`` (models/gpt_oss/modeling_gpt_oss.py:90-114, ``_apply_gate``
  :82-88): the same torch ops in the same order, bf16 throughout, ``index_add_`` in bf16 over
  the hit experts in ascending order. Expert ids outside [0, E) are skipped, as the reference's
  CUDA op does (src/kops/cohere2_moe_experts/csrc/cohere2_moe_experts.cu:35,49).
* ``experts_fp64``   — the same mathematics with every operand upcast to float64 and no
  intermediate rounding: the exact value of the op on the given bf16 inputs.
* ``route_reference`` — offsets / permutation / tile list in op_eager order, by the closed form
  ``argsort(index.T.flatten(), stable)`` and ``bincount`` (numpy).
* ``router_logits`` / ``router_select`` — the routers the reference's gpt-oss and qwen3 loaders run
  in their timed ops: transformers ``GptOssTopKRouter`` (models/gpt_oss/modeling_gpt_oss.py:126-130)
  and ``Qwen3NextTopKRouter`` (models/qwen3_next/modeling_qwen3_next.py:766-775). Logits are the
  exact (float64) value of ``x Wᵀ + b`` rounded once to bf16; selection uses a stable descending
  sort, so equal scores go to the lower expert id.

Parity pins (tests/test_oracle.py): ``router_select`` equals the routers' own code (restated as
cernels_amd.configs.modules.{GptOssRouter, Qwen3NextRouter}) on tie-free logits, and the closed
forms k = E (softmax of every logit) and k = 1 (argmax, weight 1 after renormalisation);
``experts_eager`` equals transformers' own forward bit for
bit on the committed golden fixtures (tests/golden/, written by tests/golden/make_golden.py);
``experts_fp64`` equals a per-(token, slot) brute-force loop and the closed-form special cases
(E=1,k=1 dense MLP; zero weights; gpt-oss clamps; relabelling invariance; linearity);
``route_reference`` equals the golden ``torch.where`` order and the C restatement oracle/route.c.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

LAYOUT_CONCAT = "concat"
LAYOUT_INTERLEAVED = "interleaved"
ACT_SILU = "silu"
ACT_GPTOSS = "gptoss"
GPTOSS_ALPHA = 1.702
GPTOSS_LIMIT = 7.0


def gptoss_gate(gate_up: torch.Tensor) -> torch.Tensor:
    """GptOssExperts._apply_gate (modeling_gpt_oss.py:82-88)."""
    gate, up = gate_up[..., ::2], gate_up[..., 1::2]
    gate = gate.clamp(min=None, max=GPTOSS_LIMIT)
    up = up.clamp(min=-GPTOSS_LIMIT, max=GPTOSS_LIMIT)
    glu = gate * torch.sigmoid(gate * GPTOSS_ALPHA)
    return (up + 1) * glu


def _valid_mask_index(top_k_index: torch.Tensor, E: int) -> torch.Tensor:
    """Map out-of-range ids to E (a class the loop skips, like transformers' `== num_experts`)."""
    idx = top_k_index.to(torch.int64)
    return torch.where((idx >= 0) & (idx < E), idx, torch.full_like(idx, E))


def experts_eager(x, top_k_index, top_k_weights, gate_up_proj, down_proj, gate_up_bias=None, down_bias=None,
                  layout=LAYOUT_CONCAT, act=ACT_SILU):
    """op_eager restatement on whatever device/dtype the inputs have (bf16 on CPU for parity)."""
    E = gate_up_proj.shape[0]
    final = torch.zeros_like(x)
    with torch.no_grad():
        idx = _valid_mask_index(top_k_index, E)
        expert_mask = F.one_hot(idx, num_classes=E + 1).permute(2, 1, 0)
        expert_hit = torch.greater(expert_mask.sum(dim=(-1, -2)), 0).nonzero()
        for expert_idx in expert_hit:
            expert_idx = expert_idx[0]
            if expert_idx == E:
                continue
            top_k_pos, token_idx = torch.where(expert_mask[expert_idx])
            cur = x[token_idx]
            if layout == LAYOUT_CONCAT:
                gu = F.linear(cur, gate_up_proj[expert_idx])
                if gate_up_bias is not None:
                    gu = gu + gate_up_bias[expert_idx]
                if act == ACT_SILU:
                    gate, up = gu.chunk(2, dim=-1)
                    h = F.silu(gate) * up
                else:  # gpt-oss gate on the concat layout: gate/up halves
                    gate, up = gu.chunk(2, dim=-1)
                    h = gptoss_gate(torch.stack((gate, up), dim=-1).flatten(-2))
                h = F.linear(h, down_proj[expert_idx])
            else:
                gu = cur @ gate_up_proj[expert_idx]
                if gate_up_bias is not None:
                    gu = gu + gate_up_bias[expert_idx]
                if act == ACT_GPTOSS:
                    h = gptoss_gate(gu)
                else:
                    gate, up = gu[..., ::2], gu[..., 1::2]
                    h = F.silu(gate) * up
                h = h @ down_proj[expert_idx]
            if down_bias is not None:
                h = h + down_bias[expert_idx]
            h = h * top_k_weights[token_idx, top_k_pos, None]
            final.index_add_(0, token_idx, h.to(final.dtype))
    return final


def experts_fp64(x, top_k_index, top_k_weights, gate_up_proj, down_proj, gate_up_bias=None, down_bias=None,
                 layout=LAYOUT_CONCAT, act=ACT_SILU):
    """Exact value on the given inputs: float64 everywhere, no intermediate rounding. Returns fp64."""
    d = torch.float64
    x, w = x.to(d), top_k_weights.to(d)
    E = gate_up_proj.shape[0]
    out = torch.zeros(x.shape, dtype=d, device=x.device)
    idx = _valid_mask_index(top_k_index, E)
    for e in torch.unique(idx).tolist():
        if e == E:
            continue
        tpos, kpos = torch.where(idx == e)
        cur = x[tpos]
        W1 = gate_up_proj[e].to(d)
        gu = cur @ (W1.T if layout == LAYOUT_CONCAT else W1)
        if gate_up_bias is not None:
            gu = gu + gate_up_bias[e].to(d)
        if layout == LAYOUT_CONCAT:
            gate, up = gu.chunk(2, dim=-1)
        else:
            gate, up = gu[..., ::2], gu[..., 1::2]
        if act == ACT_SILU:
            h = F.silu(gate) * up
        else:
            h = gptoss_gate(torch.stack((gate, up), dim=-1).flatten(-2))
        W2 = down_proj[e].to(d)
        y = h @ (W2.T if layout == LAYOUT_CONCAT else W2)
        if down_bias is not None:
            y = y + down_bias[e].to(d)
        out.index_add_(0, tpos, y * w[tpos, kpos, None])
    return out


def route_reference(top_k_index, num_experts: int, tile_m: int = 128) -> dict[str, np.ndarray]:
    """Closed-form routing in op_eager order.

    offsets = [0] + cumsum(bincount(valid ids)); sorted_pairs = pair ids p = t*K + k ordered by
    (expert, k, t) = stable argsort of index.T.flatten() (modeling_cohere2_moe.py:122-130 reads
    the [K, T] one-hot slice row-major); tiles = ceil(count_e / tile_m) per expert.
    """
    idx = np.asarray(top_k_index, dtype=np.int64)
    T, K = idx.shape
    flat_kt = idx.T.reshape(-1)  # slot-major: q = k*T + t
    valid = (flat_kt >= 0) & (flat_kt < num_experts)
    q = np.nonzero(valid)[0]
    order = q[np.argsort(flat_kt[q], kind="stable")]
    k_of, t_of = order // T, order % T
    sorted_pairs = (t_of * K + k_of).astype(np.int32)
    counts = np.bincount(flat_kt[valid], minlength=num_experts).astype(np.int64)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    ntiles = -(-counts // tile_m)
    tile_offsets = np.concatenate([[0], np.cumsum(ntiles)]).astype(np.int32)
    tile_expert = np.repeat(np.arange(num_experts, dtype=np.int32), ntiles)
    return {
        "offsets": offsets,
        "sorted_pairs": sorted_pairs,
        "tile_offsets": tile_offsets,
        "tile_expert": tile_expert,
        "num_tiles": int(tile_offsets[-1]),
        "num_valid": int(offsets[-1]),
    }


ROUTER_SOFTMAX_TOPK = 0  # Qwen3NextTopKRouter (renormalised when renorm=True)
ROUTER_TOPK_SOFTMAX = 1  # GptOssTopKRouter


def router_logits(x, weight, bias=None) -> torch.Tensor:
    """bf16(x Wᵀ + b): the float64 value of the bf16 inputs, rounded once (F.linear's output dtype)."""
    z = x.double() @ weight.double().T
    if bias is not None:
        z = z + bias.double()
    return z.to(torch.bfloat16)


def router_select(logits, top_k: int, mode: int, renorm: bool = True):
    """(indices int64 [T,k], weights bf16 [T,k]) from bf16 logits [T,E], ties to the lower id.

    SOFTMAX_TOPK (modeling_qwen3_next.py:769-773): softmax in fp32, top-k, renormalise, bf16.
    TOPK_SOFTMAX (modeling_gpt_oss.py:128-129): top-k of the logits, softmax over them, bf16.
    Both choose the experts on the logits: softmax is strictly increasing, so the top-k of the
    probabilities is the top-k of the logits, and equal probabilities come only from equal logits.
    (Choosing on fp32 probabilities instead would let the rounding of exp tie two distinct logits.)
    """
    lf = logits.float()
    if mode == ROUTER_SOFTMAX_TOPK:
        probs = torch.softmax(lf, dim=-1, dtype=torch.float32)
        _, order = torch.sort(lf, dim=-1, descending=True, stable=True)
        idx = order[:, :top_k]
        w = torch.gather(probs, 1, idx)
        if renorm:
            w = w / w.sum(dim=-1, keepdim=True)
    elif mode == ROUTER_TOPK_SOFTMAX:
        vals, order = torch.sort(lf, dim=-1, descending=True, stable=True)
        idx = order[:, :top_k]
        w = torch.softmax(vals[:, :top_k], dim=-1, dtype=torch.float32)
    else:
        raise ValueError(f"unknown router mode {mode}")
    return idx, w.to(torch.bfloat16)


MEGABLOCKS_ACT_FNS = {0: lambda h: F.gelu(h, approximate="tanh"), 1: F.silu, 2: F.relu}


def megablocks_fp64(x, top_k_index, top_k_weights, w1, w2, act_id: int):
    """megablocks_moe (src/kops/megablocks_moe/csrc/megablocks_moe.cu:141-254): for every (token, slot)
    with expert id e in [0, E) (.cu:32,56), ``weight * act(x w1[e]) w2[e]`` summed per token; w1 is
    [E, H, F], w2 [E, F, H]; act_id 0 = GELU tanh form (.cu:81-84), 1 = SiLU, 2 = ReLU (.cu:86-96).
    Float64 with no intermediate rounding (the reference rounds both GEMM outputs to bf16). Returns
    fp64 [T, H]."""
    d = torch.float64
    act = MEGABLOCKS_ACT_FNS[int(act_id)]
    x, w = x.to(d), top_k_weights.to(d)
    E = w1.shape[0]
    out = torch.zeros(x.shape, dtype=d, device=x.device)
    idx = _valid_mask_index(top_k_index, E)
    for e in torch.unique(idx).tolist():
        if e == E:
            continue
        tpos, kpos = torch.where(idx == e)
        y = act(x[tpos] @ w1[e].to(d)) @ w2[e].to(d)
        out.index_add_(0, tpos, y * w[tpos, kpos, None])
    return out


def shared_expert_fp64(x, gate_proj, up_proj, down_proj, shared_gate):
    """``sigmoid(shared_expert_gate(x)) * shared_expert(x)`` of Qwen3NextSparseMoeBlock
    (transformers/models/qwen3_next/modeling_qwen3_next.py:789-795, Qwen3NextMLP :730-745 style
    ``down(silu(gate x) * up x)``). The gate logit and its sigmoid are rounded to bf16, as the bf16
    ``nn.Linear`` and ``torch.sigmoid`` produce them; the MLP is float64 with no intermediate
    rounding. Returns fp64 [T, H]."""
    d = torch.float64
    xd = x.to(d)
    logit = (xd @ shared_gate.to(d).T).to(torch.bfloat16)
    s = torch.sigmoid(logit.to(d)).to(torch.bfloat16).to(d)
    h = F.silu(xd @ gate_proj.to(d).T) * (xd @ up_proj.to(d).T)
    return s * (h @ down_proj.to(d).T)


def error_stats(out: torch.Tensor, ref: torch.Tensor) -> dict[str, float]:
    """max |out - ref| and RMS(ref) (both fp64); the bar is max_abs <= 2e-2 * rms."""
    o, r = out.double().cpu(), ref.double().cpu()
    rms = float(r.pow(2).mean().sqrt()) if r.numel() else 0.0
    mx = float((o - r).abs().max()) if r.numel() else 0.0
    return {"max_abs": mx, "rms_ref": rms, "ratio": mx / rms if rms > 0 else (0.0 if mx == 0 else float("inf"))}
