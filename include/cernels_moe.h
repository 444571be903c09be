/*
 * cernels_moe.h — C ABI of the MI355X (gfx950) routed MoE-experts library, libcernels_moe.so.
 *
 * Plain pointers and sizes only; no torch types. Every entry point is asynchronous on the
 * caller's HIP stream, performs no host synchronisation and allocates no device memory: the
 * caller passes a workspace of at least the size the matching *_workspace_bytes() returns.
 * All return a status (CERNELS_MOE_OK = 0); cernels_moe_status_string() names it.
 *
 * Tensor conventions (all row-major, contiguous, 16-byte aligned):
 *   x              [T, H]   bf16         hidden states
 *   indices        [T, K]   int32        top_k_index (expert id per token and slot)
 *   weights        [T, K]   fp32         top_k_weights (routing weight per token and slot)
 *   out            [T, H]   bf16         written in full
 *   layout CONCAT:      gate_up_proj [E, 2F, H] (rows 0..F-1 gate, F..2F-1 up), down_proj [E, H, F]
 *   layout INTERLEAVED: gate_up_proj [E, H, 2F] (even columns gate, odd up),   down_proj [E, F, H]
 *   gate_up_bias   [E, 2F]  fp32 or NULL (same column order as the layout)
 *   down_bias      [E, H]   fp32 or NULL
 * Expert ids outside [0, E) contribute nothing (as the reference prefill op,
 * src/kops/cohere2_moe_experts/csrc/cohere2_moe_experts.cu:35,49).
 *
 * Reference interface replaced: the torch ops registered in
 *   src/kops/cohere2_moe_experts/torch-ext/torch_binding.cpp:6-13,
 *   src/kops/deepseek_ocr2_moe_experts/torch-ext/torch_binding.cpp,
 *   src/kops/qwen3_next_moe_experts/torch-ext/torch_binding.cpp,
 *   src/kops/gpt_oss_moe_experts/torch-ext/torch_binding.cpp:7-10
 * whose C++ signatures are in the matching torch-ext/torch_binding.h.
 */
#ifndef CERNELS_MOE_H
#define CERNELS_MOE_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum cernels_moe_status {
    CERNELS_MOE_OK = 0,
    CERNELS_MOE_INVALID_ARGUMENT = 1,   /* null pointer, negative or zero dimension, bad enum */
    CERNELS_MOE_UNSUPPORTED_SHAPE = 2,  /* shape outside what the kernels handle (see each entry) */
    CERNELS_MOE_MISALIGNED = 3,         /* a tensor pointer is not 16-byte aligned */
    CERNELS_MOE_WORKSPACE_TOO_SMALL = 4,
    CERNELS_MOE_HIP_ERROR = 5           /* a kernel launch failed */
};

enum cernels_moe_layout { CERNELS_MOE_LAYOUT_CONCAT = 0, CERNELS_MOE_LAYOUT_INTERLEAVED = 1 };
enum cernels_moe_act {
    CERNELS_MOE_ACT_SILU = 0,       /* silu(gate) * up */
    CERNELS_MOE_ACT_GPTOSS = 1,     /* (clamp(up,-7,7) + 1) * g * sigmoid(1.702 g), g = min(gate, 7) */
    /* non-gated (one first projection H -> F, megablocks_moe; packed entries only, no first-projection bias): */
    CERNELS_MOE_ACT_GELU_TANH = 2,  /* 0.5 h (1 + tanh(sqrt(2/pi) (h + 0.044715 h^3))) */
    CERNELS_MOE_ACT_SILU_PLAIN = 3, /* h sigmoid(h) */
    CERNELS_MOE_ACT_RELU = 4        /* max(h, 0) */
};

/* GATE_UP: gated first projection; DOWN: second projection; UP: non-gated first projection. */
enum cernels_moe_projection { CERNELS_MOE_GATE_UP = 0, CERNELS_MOE_DOWN = 1, CERNELS_MOE_UP = 2 };

const char* cernels_moe_version(void);
const char* cernels_moe_status_string(int status);

/* ---- routing (prefill): histogram -> offsets -> stable permutation -> M-tile list ---------------
 * Replaces count_tokens_kernel + at::cumsum + build_perm_kernel
 * (src/kops/cohere2_moe_experts/csrc/cohere2_moe_experts.cu:29-55, :262-284).
 *   expert_offsets [E+1]: exclusive scan of per-expert pair counts; expert_offsets[E] = valid pairs.
 *   sorted_pairs   [T*K]: pair ids p = t*K + k grouped by expert, within an expert by slot k then
 *                         token t (the op_eager order); entries past expert_offsets[E] are unset.
 *   tile_offsets   [E+1]: exclusive scan of ceil(count_e / tile_m).
 *   tile_expert    [cernels_moe_route_tile_capacity()]: expert of each M-tile.
 *   meta           [2]  : meta[0] = number of M-tiles, meta[1] = valid pairs.
 *   workspace      scratch of cernels_moe_route_workspace_bytes() (per-tile expert counts).
 * Limits: 1 <= E <= 1024, 1 <= K <= 4096, T*K < 2^31, tile_m >= 1. */
size_t cernels_moe_route_tile_capacity(int32_t T, int32_t K, int32_t E, int32_t tile_m);
size_t cernels_moe_route_workspace_bytes(int32_t T, int32_t K, int32_t E);
int cernels_moe_route(const int32_t* indices, int32_t T, int32_t K, int32_t E, int32_t tile_m,
                      int32_t* expert_offsets, int32_t* sorted_pairs, int32_t* tile_offsets,
                      int32_t* tile_expert, int32_t* meta, void* workspace, size_t workspace_bytes,
                      hipStream_t stream);

/* ---- prefill: grouped GEMM experts ------------------------------------------------------------
 * route -> gate_up GEMM (+bias, SwiGLU in the epilogue) -> down GEMM (+bias, x routing weight in
 * the epilogue) -> deterministic top-k combine. Any T >= 0 (T = 0 is a no-op).
 * Limits: H % 64 == 0, F % 64 == 0, E <= 1024, K <= 4096. */
size_t cernels_moe_experts_workspace_bytes(int32_t T, int32_t H, int32_t F, int32_t E, int32_t K);
int cernels_moe_experts(const void* x, const void* gate_up_proj, const float* gate_up_bias,
                        const void* down_proj, const float* down_bias, const int32_t* indices,
                        const float* weights, int32_t T, int32_t H, int32_t F, int32_t E, int32_t K,
                        int32_t layout, int32_t act, void* out, void* workspace, size_t workspace_bytes,
                        hipStream_t stream);

/* Same as cernels_moe_experts, and, when stage_events is not NULL, records 5 caller-created
 * events on `stream`: before routing, after routing, after the gate_up GEMM, after the down GEMM
 * and after the combine (per-stage timing; no work is skipped). No counterpart in the reference. */
int cernels_moe_experts_staged(const void* x, const void* gate_up_proj, const float* gate_up_bias,
                               const void* down_proj, const float* down_bias, const int32_t* indices,
                               const float* weights, int32_t T, int32_t H, int32_t F, int32_t E, int32_t K,
                               int32_t layout, int32_t act, void* out, void* workspace, size_t workspace_bytes,
                               hipStream_t stream, hipEvent_t* stage_events);

/* ---- prefill on packed expert weights ------------------------------------------------------------
 * The same operation as cernels_moe_experts, on weights re-laid once by cernels_moe_pack_weights
 * into MFMA-fragment order (each 32x16 operand fragment is 1 KB of contiguous memory in the order
 * a 64-lane wave reads it). A model packs its expert weights once at load time, as the reference's
 * gpt-oss loader caches converted copies of its expert tensors (src/kops/registry/gpt_oss_moe_experts.py:14-26);
 * every later call streams them sequentially. GATE_UP and UP keep bf16 and the element count (2FH
 * and HF per expert). DOWN is stored as fp16 (the second projection multiplies fp16 activations,
 * 2^-11 rounding instead of bf16's 2^-8), each 32-output-column fragment scaled by a power of two
 * so its largest |w| lies in [2^14, 2^15); the fp16 fragments (HF per expert) are followed by a
 * table of those powers (one int8 per expert and fragment, padded to 256 bytes). Size with
 * cernels_moe_packed_weight_bytes. Either source layout is accepted; the packed format does not
 * depend on it. No counterpart op in the reference: these entries are the fast path behind the
 * same loaders.
 *   which: CERNELS_MOE_GATE_UP (src [E,2F,H] concat or [E,H,2F] interleaved), CERNELS_MOE_DOWN
 *          (src [E,H,F] concat or [E,F,H] interleaved) or CERNELS_MOE_UP (non-gated first projection,
 *          src [E,F,H] concat or [E,H,F] interleaved, i.e. megablocks' w1).
 *   act: a non-gated act (GELU_TANH, SILU_PLAIN, RELU) takes gate_up_packed packed as CERNELS_MOE_UP
 *          and no gate_up_bias.
 *   bias_layout (experts_packed): column order of gate_up_bias, CERNELS_MOE_LAYOUT_CONCAT
 *          ([gate F | up F]) or CERNELS_MOE_LAYOUT_INTERLEAVED (gate/up alternating).
 * Limits: H % 64 == 0, F % 64 == 0, E <= 1024, K <= 4096; experts_packed also T*H*2 < 2^31 (32-bit offsets).
 * Otherwise CERNELS_MOE_UNSUPPORTED_SHAPE. */
size_t cernels_moe_packed_weight_bytes(int32_t H, int32_t F, int32_t E, int32_t which);
int cernels_moe_pack_weights(const void* src, int32_t H, int32_t F, int32_t E, int32_t layout, int32_t which,
                             void* dst, hipStream_t stream);
int cernels_moe_experts_packed(const void* x, const void* gate_up_packed, const float* gate_up_bias,
                               const void* down_packed, const float* down_bias, const int32_t* indices,
                               const float* weights, int32_t T, int32_t H, int32_t F, int32_t E, int32_t K,
                               int32_t bias_layout, int32_t act, void* out, void* workspace, size_t workspace_bytes,
                               hipStream_t stream);
/* With 5 stage events, as cernels_moe_experts_staged. */
int cernels_moe_experts_packed_staged(const void* x, const void* gate_up_packed, const float* gate_up_bias,
                                      const void* down_packed, const float* down_bias, const int32_t* indices,
                                      const float* weights, int32_t T, int32_t H, int32_t F, int32_t E, int32_t K,
                                      int32_t bias_layout, int32_t act, void* out, void* workspace,
                                      size_t workspace_bytes, hipStream_t stream, hipEvent_t* stage_events);

/* ---- decode: fused gather-GEMV over the distinct selected experts -------------------------------
 * Two launches, no atomics on the output, no host sync. Layout CONCAT only.
 * Limits: T <= cernels_moe_decode_max_tokens(), T*K <= cernels_moe_decode_max_pairs(),
 * H % 8 == 0, F % 8 == 0, H <= 4096, F <= 4096. */
int32_t cernels_moe_decode_max_tokens(void);
int32_t cernels_moe_decode_max_pairs(void);
size_t cernels_moe_experts_decode_workspace_bytes(int32_t T, int32_t H, int32_t F, int32_t E, int32_t K);
int cernels_moe_experts_decode(const void* x, const void* gate_up_proj, const float* gate_up_bias,
                               const void* down_proj, const float* down_bias, const int32_t* indices,
                               const float* weights, int32_t T, int32_t H, int32_t F, int32_t E, int32_t K,
                               int32_t layout, int32_t act, void* out, void* workspace,
                               size_t workspace_bytes, hipStream_t stream);

/* Decode with 3 stage events (before gate_up, after gate_up, after down) when not NULL. */
int cernels_moe_experts_decode_staged(const void* x, const void* gate_up_proj, const float* gate_up_bias,
                                      const void* down_proj, const float* down_bias, const int32_t* indices,
                                      const float* weights, int32_t T, int32_t H, int32_t F, int32_t E, int32_t K,
                                      int32_t layout, int32_t act, void* out, void* workspace,
                                      size_t workspace_bytes, hipStream_t stream, hipEvent_t* stage_events);

/* Allocation-free decode. No counterpart in the reference: for callers that cannot allocate device
 * memory or pass a workspace (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Same arguments and result as cernels_moe_experts_decode without the workspace:
 * the library keeps one static scratch of CERNELS_MOE_DECODE_NOALLOC_SCRATCH_BYTES per GPU (held
 * until the process ends) and calls no allocating routine. Every shape the decode entry accepts
 * fits it (T*K <= cernels_moe_decode_max_pairs(), F <= 4096); a larger workspace need returns
 * CERNELS_MOE_WORKSPACE_TOO_SMALL. Calls that overlap on one GPU share the scratch and race:
 * serialise them (one stream, or events). */
#define CERNELS_MOE_DECODE_NOALLOC_SCRATCH_BYTES (256u * 4096u * 2u + 256u * 4u)
int cernels_moe_experts_decode_noalloc(const void* x, const void* gate_up_proj, const float* gate_up_bias,
                                       const void* down_proj, const float* down_bias, const int32_t* indices,
                                       const float* weights, int32_t T, int32_t H, int32_t F, int32_t E, int32_t K,
                                       int32_t layout, int32_t act, void* out, hipStream_t stream);

/* ---- router -------------------------------------------------------------------------------------
 * logits = bf16(x W^T + b) for x [T, H] bf16, W [E, H] bf16, b [E] bf16 (nullable), then per token:
 *   CERNELS_MOE_ROUTER_SOFTMAX_TOPK: softmax over the E logits in fp32, the K largest probabilities,
 *       renormalised to sum 1 if renorm != 0 (transformers Qwen3NextTopKRouter,
 *       modeling_qwen3_next.py:766-775);
 *   CERNELS_MOE_ROUTER_TOPK_SOFTMAX: the K largest logits, softmax over those K values
 *       (transformers GptOssTopKRouter, modeling_gpt_oss.py:126-130).
 * Writes indices [T, K+S] int32 (descending by score; ties to the lower expert id) and weights
 * [T, K+S] fp32 holding the bf16-rounded scores, i.e. what the experts entries take, and logits
 * [T, E'] bf16 (required: the routers return them too, and for E' > 64 they carry the logits from the
 * GEMM kernel to the selection kernel). Replaces the module routers the reference's gpt-oss and qwen3
 * loaders call inside their timed ops (src/kops/registry/gpt_oss_moe_experts.py:35,
 * src/kops/registry/qwen3_next_moe_experts.py:28).
 * Shared expert (shared_slots = S > 0, Qwen3NextSparseMoeBlock, modeling_qwen3_next.py:789-795): W and
 * b have E' = E + 1 rows, the last being shared_expert_gate's weight; slots K..K+S-1 of every token get
 * ids E..E+S-1 and weight bf16(sigmoid(logit E)). With the shared expert's MLP packed as experts
 * E..E+S-1 (its intermediate split into S blocks of F), the experts op then adds
 * sigmoid(x g) * shared_expert(x) to the routed sum. S = 0: E' = E and K slots.
 * Limits: 1 <= K <= min(E, 32), 0 <= S <= 32, E' <= 1024, H % 16 == 0; x and W 16-byte aligned. */
enum cernels_moe_router_mode { CERNELS_MOE_ROUTER_SOFTMAX_TOPK = 0, CERNELS_MOE_ROUTER_TOPK_SOFTMAX = 1 };
int cernels_moe_router(const void* x, const void* router_weight, const void* router_bias, int32_t T, int32_t H,
                       int32_t E, int32_t K, int32_t mode, int32_t renorm, int32_t shared_slots, int32_t* indices,
                       float* weights, void* logits, hipStream_t stream);

/* ---- megablocks_moe (src/kops/megablocks_moe/torch-ext/torch_binding.cpp; csrc/megablocks_moe.cu:141-254) --
 * Non-gated experts: out = sum_k w_k * act(x W1[e_k]) W2[e_k], x [T,H], w1 [E,H,F], w2 [E,F,H] bf16,
 * indices [T,topk] int32, weights [T,topk] fp32, act_id 0 = GELU (tanh form), 1 = SiLU, 2 = ReLU, as
 * the reference op's. The weights are packed into the workspace on every call (the reference op
 * also takes the weights as stored); a caller that keeps them resident packs once with
 * cernels_moe_pack_weights (CERNELS_MOE_UP / CERNELS_MOE_DOWN, interleaved layout) and calls
 * cernels_moe_experts_packed, as the megablocks loader here does.
 * Limits: H % 64 == 0, F % 64 == 0, E <= 1024, topk <= 4096, T*H*2 < 2^31. */
size_t cernels_megablocks_moe_workspace_bytes(int32_t T, int32_t H, int32_t F, int32_t E, int32_t topk);
int cernels_megablocks_moe(const void* x, const void* w1, const void* w2, const int32_t* indices, const float* weights,
                           int32_t T, int32_t H, int32_t F, int32_t E, int32_t topk, int32_t act_id, void* out,
                           void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---- the reference's per-model ops, same argument order as their torch schemas ----------------
 * cohere2_moe_experts(Tensor x, Tensor gate_up_proj, Tensor down_proj, Tensor indices,
 *                     Tensor weights, int topk) -> Tensor
 *   (src/kops/cohere2_moe_experts/torch-ext/torch_binding.cpp:7-9; .cu:238-361)
 * cohere2_moe_experts_decode(...)            (torch_binding.cpp:10-12; .cu:199-236)
 * deepseek_ocr2_moe_experts(...) / _decode   (src/kops/deepseek_ocr2_moe_experts/csrc/
 *                                             deepseek_ocr2_moe_experts.cu:240-363 / :201-238)
 * qwen3_next_moe_experts(...)                (src/kops/qwen3_next_moe_experts/csrc/
 *                                             qwen3_next_moe_experts.cu:97-220)
 * Concat layout, SiLU; T, H, F, E come from the tensor shapes on the torch side. */
int cernels_cohere2_moe_experts(const void* x, const void* gate_up_proj, const void* down_proj,
                                const int32_t* indices, const float* weights, int32_t T, int32_t H,
                                int32_t F, int32_t E, int32_t topk, void* out, void* workspace,
                                size_t workspace_bytes, hipStream_t stream);
int cernels_cohere2_moe_experts_decode(const void* x, const void* gate_up_proj, const void* down_proj,
                                       const int32_t* indices, const float* weights, int32_t T,
                                       int32_t H, int32_t F, int32_t E, int32_t topk, void* out,
                                       void* workspace, size_t workspace_bytes, hipStream_t stream);
int cernels_deepseek_ocr2_moe_experts(const void* x, const void* gate_up_proj, const void* down_proj,
                                      const int32_t* indices, const float* weights, int32_t T,
                                      int32_t H, int32_t F, int32_t E, int32_t topk, void* out,
                                      void* workspace, size_t workspace_bytes, hipStream_t stream);
int cernels_deepseek_ocr2_moe_experts_decode(const void* x, const void* gate_up_proj,
                                             const void* down_proj, const int32_t* indices,
                                             const float* weights, int32_t T, int32_t H, int32_t F,
                                             int32_t E, int32_t topk, void* out, void* workspace,
                                             size_t workspace_bytes, hipStream_t stream);
int cernels_qwen3_next_moe_experts(const void* x, const void* gate_up_proj, const void* down_proj,
                                   const int32_t* indices, const float* weights, int32_t T, int32_t H,
                                   int32_t F, int32_t E, int32_t topk, void* out, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream);
/* gpt_oss_moe_experts(Tensor x, Tensor gate_up_proj, Tensor gate_up_bias, Tensor down_proj,
 *                     Tensor down_bias, Tensor indices, Tensor weights, int topk) -> Tensor
 *   (src/kops/gpt_oss_moe_experts/torch-ext/torch_binding.cpp:7-10; .cu:119-245)
 * Interleaved layout, fp32 biases, clamped SwiGLU. */
int cernels_gpt_oss_moe_experts(const void* x, const void* gate_up_proj, const float* gate_up_bias,
                                const void* down_proj, const float* down_bias, const int32_t* indices,
                                const float* weights, int32_t T, int32_t H, int32_t F, int32_t E,
                                int32_t topk, void* out, void* workspace, size_t workspace_bytes,
                                hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* CERNELS_MOE_H */
