// extern "C" entry points of libcernels_moe.so (declared in include/cernels_moe.h).
// Argument checking, workspace carving and kernel sequencing; no device allocation, no host sync.
#include <hip/hip_runtime.h>

#include <cstdint>

#include <algorithm>

#include "../../include/cernels_moe.h"

namespace cmoe {
struct GemmParams;
struct XcdSplit;
hipError_t launch_route(const int32_t* idx, int T, int K, int E, int BM, int32_t* offsets, int32_t* sorted_pairs,
                        int32_t* tile_offsets, int32_t* tile_expert, int32_t* meta, int32_t* counts,
                        int32_t* sched, hipStream_t stream, int8_t* row_zero = nullptr,
                        const XcdSplit* split = nullptr);
size_t route_workspace_bytes(int T, int K, int E);
int gemm_tile_m();
int packed_tile_m();
int router_max_experts();
int router_max_topk();
hipError_t launch_router(const uint16_t* x, const uint16_t* w, const uint16_t* bias, int T, int H, int E, int K,
                         int mode, int renorm, int S, int32_t* idx, float* wt, uint16_t* logits, hipStream_t s);
hipError_t launch_prefill(const void* x, const void* w1, const float* b1, const void* w2, const float* b2,
                          const int32_t* idx, const float* route_w, int T, int H, int F, int E, int K, int layout,
                          int act, void* out, int32_t* offsets, int32_t* tile_offsets, int32_t* meta,
                          int32_t* sorted_pairs, int32_t* tile_expert, int32_t* route_counts, int max_tiles,
                          uint16_t* glu, float* Y, hipStream_t s, hipEvent_t* ev);
bool decode_shape_supported(int H, int F);
size_t decode_noalloc_bytes();
hipError_t decode_noalloc_scratch(void** ptr);
int decode_max_pairs();
int decode_max_tokens();
size_t packed_weight_bytes(int H, int F, int E, int which);
hipError_t launch_pack(const uint16_t* src, uint16_t* dst, int E, int H, int F, int layout, int which, hipStream_t s);
hipError_t launch_prefill_packed(const void* x, const void* w1p, const float* b1, const void* w2p, const float* b2,
                                 const int32_t* idx, const float* route_w, int T, int H, int F, int E, int K,
                                 int bias_interleaved, int act, void* out, int32_t* offsets, int32_t* tile_offsets,
                                 int32_t* meta, int32_t* sorted_pairs, int32_t* tile_expert, int32_t* route_counts,
                                 int max_tiles, uint16_t* glu, float* Y, int8_t* gexp, int8_t* rsig,
                                 int8_t* psig, hipStream_t s, hipEvent_t* ev);
hipError_t launch_decode(const uint16_t* x, const uint16_t* w1, const float* b1, const uint16_t* w2, const float* b2,
                         const int32_t* idx, const float* route_w, uint16_t* glu, int32_t* order, uint16_t* out,
                         int T, int H, int F, int E, int K, int act, hipStream_t s, hipEvent_t* ev);
}  // namespace cmoe

namespace {

constexpr int kMaxExperts = 1024;
constexpr size_t kAlign = 256;

size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct PrefillWs {
    size_t offsets, tile_offsets, meta, sorted_pairs, tile_expert, route_counts, glu, Y, gexp, rsig, psig, total;
    int capacity;
};

PrefillWs prefill_ws(int T, int H, int F, int E, int K) {
    PrefillWs w{};
    const long long P = (long long)T * K;
    const int bm = std::min(cmoe::gemm_tile_m(), cmoe::packed_tile_m());  // M-tile list sized for either GEMM
    w.capacity = (int)((P + bm - 1) / bm + (P < E ? P : E));
    size_t o = 0;
    w.offsets = o;      o = align_up(o + sizeof(int32_t) * (E + 1));
    w.tile_offsets = o; o = align_up(o + sizeof(int32_t) * (E + 1));
    w.meta = o;         o = align_up(o + sizeof(int32_t) * 64);  // [0..1] route totals, [8..31] GEMM counters, flags,
                                                                 // [32..49] per-XCD item ranges (packed)
    w.sorted_pairs = o; o = align_up(o + sizeof(int32_t) * P);
    w.tile_expert = o;  o = align_up(o + sizeof(int32_t) * (size_t)(w.capacity > 0 ? w.capacity : 1));
    w.route_counts = o; o = align_up(o + cmoe::route_workspace_bytes(T, K, E));
    w.glu = o;          o = align_up(o + sizeof(uint16_t) * 2 * P * F);  // stored layout: bf16 pairs; packed: fp16
    w.Y = o;            o = align_up(o + 3 * P * H);  // 24-bit floats (both paths)
    w.gexp = o;         o = align_up(o + (size_t)P * (F / 16));  // packed path: exponent per 16-column glu segment
    w.rsig = o;         o = align_up(o + (size_t)P);             // packed path: per glu row scale
    w.psig = o;         o = align_up(o + (size_t)P);             // packed path: the same, per pair
    w.total = o;
    return w;
}

struct DecodeWs {
    size_t glu, order, total;
};

DecodeWs decode_ws(int T, int H, int F, int K) {
    (void)H;
    DecodeWs w{};
    const long long P = (long long)T * K;
    size_t o = 0;
    w.glu = o; o = align_up(o + sizeof(uint16_t) * P * F);
    w.order = o; o = align_up(o + sizeof(int32_t) * P);  // valid pairs sorted by expert, then -1
    w.total = o;
    return w;
}

constexpr int kMaxTopk = 4096;  // the route kernels divide pair positions by T through a float reciprocal

bool dims_ok(int T, int H, int F, int E, int K) {
    return T >= 0 && H > 0 && F > 0 && E > 0 && K > 0 && K <= kMaxTopk && (long long)T * K < (1LL << 31);
}

int common_checks(const void* x, const void* w1, const void* w2, const int32_t* idx, const float* wts, int T,
                  int H, int F, int E, int K, int layout, int act, void* out, void* ws) {
    if (!dims_ok(T, H, F, E, K)) return CERNELS_MOE_INVALID_ARGUMENT;
    if (layout != CERNELS_MOE_LAYOUT_CONCAT && layout != CERNELS_MOE_LAYOUT_INTERLEAVED)
        return CERNELS_MOE_INVALID_ARGUMENT;
    if (act < CERNELS_MOE_ACT_SILU || act > CERNELS_MOE_ACT_RELU) return CERNELS_MOE_INVALID_ARGUMENT;
    if (T == 0) return CERNELS_MOE_OK;
    if (!x || !w1 || !w2 || !idx || !wts || !out || !ws) return CERNELS_MOE_INVALID_ARGUMENT;
    if (!aligned16(x) || !aligned16(w1) || !aligned16(w2) || !aligned16(out) || !aligned16(ws))
        return CERNELS_MOE_MISALIGNED;
    if ((reinterpret_cast<uintptr_t>(idx) & 3u) || (reinterpret_cast<uintptr_t>(wts) & 3u))
        return CERNELS_MOE_MISALIGNED;
    return CERNELS_MOE_OK;
}

int hip_status(hipError_t e) { return e == hipSuccess ? CERNELS_MOE_OK : CERNELS_MOE_HIP_ERROR; }

bool act_gated(int act) { return act == CERNELS_MOE_ACT_SILU || act == CERNELS_MOE_ACT_GPTOSS; }

}  // namespace

extern "C" {

const char* cernels_moe_version(void) { return "cernels_moe 0.1 gfx950"; }

const char* cernels_moe_status_string(int status) {
    switch (status) {
        case CERNELS_MOE_OK: return "ok";
        case CERNELS_MOE_INVALID_ARGUMENT: return "invalid argument";
        case CERNELS_MOE_UNSUPPORTED_SHAPE: return "unsupported shape";
        case CERNELS_MOE_MISALIGNED: return "tensor pointer not 16-byte aligned";
        case CERNELS_MOE_WORKSPACE_TOO_SMALL: return "workspace too small";
        case CERNELS_MOE_HIP_ERROR: return "HIP kernel launch failed";
        default: return "unknown status";
    }
}

size_t cernels_moe_route_workspace_bytes(int32_t T, int32_t K, int32_t E) {
    if (T < 0 || K <= 0 || E <= 0 || (long long)T * K >= (1LL << 31)) return 0;
    return cmoe::route_workspace_bytes(T, K, E);
}

size_t cernels_moe_route_tile_capacity(int32_t T, int32_t K, int32_t E, int32_t tile_m) {
    if (T < 0 || K <= 0 || E <= 0 || tile_m <= 0) return 0;
    const long long P = (long long)T * K;
    const long long cap = (P + tile_m - 1) / tile_m + (P < E ? P : E);
    return (size_t)(cap > 0 ? cap : 1);
}

int cernels_moe_route(const int32_t* indices, int32_t T, int32_t K, int32_t E, int32_t tile_m,
                      int32_t* expert_offsets, int32_t* sorted_pairs, int32_t* tile_offsets, int32_t* tile_expert,
                      int32_t* meta, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (T < 0 || K <= 0 || K > kMaxTopk || E <= 0 || E > kMaxExperts || tile_m <= 0 || (long long)T * K >= (1LL << 31))
        return CERNELS_MOE_INVALID_ARGUMENT;
    if (!expert_offsets || !tile_offsets || !tile_expert || !meta || !workspace) return CERNELS_MOE_INVALID_ARGUMENT;
    if (T > 0 && (!indices || !sorted_pairs)) return CERNELS_MOE_INVALID_ARGUMENT;
    if (workspace_bytes < cmoe::route_workspace_bytes(T, K, E)) return CERNELS_MOE_WORKSPACE_TOO_SMALL;
    return hip_status(cmoe::launch_route(indices, T, K, E, tile_m, expert_offsets, sorted_pairs, tile_offsets,
                                         tile_expert, meta, static_cast<int32_t*>(workspace), nullptr, stream));
}

int cernels_moe_router(const void* x, const void* router_weight, const void* router_bias, int32_t T, int32_t H,
                       int32_t E, int32_t K, int32_t mode, int32_t renorm, int32_t shared_slots, int32_t* indices,
                       float* weights, void* logits, hipStream_t stream) {
    if (T < 0 || H <= 0 || E <= 0 || K <= 0 || shared_slots < 0) return CERNELS_MOE_INVALID_ARGUMENT;
    if (mode != CERNELS_MOE_ROUTER_SOFTMAX_TOPK && mode != CERNELS_MOE_ROUTER_TOPK_SOFTMAX)
        return CERNELS_MOE_INVALID_ARGUMENT;
    if (T == 0) return CERNELS_MOE_OK;
    if (!x || !router_weight || !indices || !weights || !logits) return CERNELS_MOE_INVALID_ARGUMENT;
    if (K > E || K > cmoe::router_max_topk() || shared_slots > cmoe::router_max_topk() ||
        E + (shared_slots > 0) > cmoe::router_max_experts() || H % 16)
        return CERNELS_MOE_UNSUPPORTED_SHAPE;
    if (!aligned16(x) || !aligned16(router_weight)) return CERNELS_MOE_MISALIGNED;
    if ((reinterpret_cast<uintptr_t>(router_bias) & 1u) || (reinterpret_cast<uintptr_t>(logits) & 1u) ||
        (reinterpret_cast<uintptr_t>(indices) & 3u) || (reinterpret_cast<uintptr_t>(weights) & 3u))
        return CERNELS_MOE_MISALIGNED;
    return hip_status(cmoe::launch_router(static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(router_weight),
                                          static_cast<const uint16_t*>(router_bias), T, H, E, K, mode, renorm != 0,
                                          shared_slots, indices, weights, static_cast<uint16_t*>(logits), stream));
}

size_t cernels_moe_experts_workspace_bytes(int32_t T, int32_t H, int32_t F, int32_t E, int32_t K) {
    if (!dims_ok(T, H, F, E, K)) return 0;
    return prefill_ws(T, H, F, E, K).total;
}

int cernels_moe_experts_staged(const void* x, const void* gate_up_proj, const float* gate_up_bias,
                               const void* down_proj, const float* down_bias, const int32_t* indices,
                               const float* weights, int32_t T, int32_t H, int32_t F, int32_t E, int32_t K,
                               int32_t layout, int32_t act, void* out, void* workspace, size_t workspace_bytes,
                               hipStream_t stream, hipEvent_t* stage_events) {
    int st = common_checks(x, gate_up_proj, down_proj, indices, weights, T, H, F, E, K, layout, act, out, workspace);
    if (st != CERNELS_MOE_OK || T == 0) return st;
    if (!act_gated(act)) return CERNELS_MOE_UNSUPPORTED_SHAPE;  // non-gated: packed entries only
    if (H % 64 || F % 64 || E > kMaxExperts) return CERNELS_MOE_UNSUPPORTED_SHAPE;
    const PrefillWs w = prefill_ws(T, H, F, E, K);
    if (workspace_bytes < w.total) return CERNELS_MOE_WORKSPACE_TOO_SMALL;
    char* base = static_cast<char*>(workspace);
    return hip_status(cmoe::launch_prefill(
        x, gate_up_proj, gate_up_bias, down_proj, down_bias, indices, weights, T, H, F, E, K, layout, act, out,
        reinterpret_cast<int32_t*>(base + w.offsets), reinterpret_cast<int32_t*>(base + w.tile_offsets),
        reinterpret_cast<int32_t*>(base + w.meta), reinterpret_cast<int32_t*>(base + w.sorted_pairs),
        reinterpret_cast<int32_t*>(base + w.tile_expert), reinterpret_cast<int32_t*>(base + w.route_counts),
        w.capacity, reinterpret_cast<uint16_t*>(base + w.glu),
        reinterpret_cast<float*>(base + w.Y), stream, stage_events));
}

int cernels_moe_experts(const void* x, const void* gate_up_proj, const float* gate_up_bias, const void* down_proj,
                        const float* down_bias, const int32_t* indices, const float* weights, int32_t T, int32_t H,
                        int32_t F, int32_t E, int32_t K, int32_t layout, int32_t act, void* out, void* workspace,
                        size_t workspace_bytes, hipStream_t stream) {
    return cernels_moe_experts_staged(x, gate_up_proj, gate_up_bias, down_proj, down_bias, indices, weights, T, H, F,
                                      E, K, layout, act, out, workspace, workspace_bytes, stream, nullptr);
}

// ---- packed weights ------------------------------------------------------------------------------

size_t cernels_moe_packed_weight_bytes(int32_t H, int32_t F, int32_t E, int32_t which) {
    if (H <= 0 || F <= 0 || E <= 0 || which < CERNELS_MOE_GATE_UP || which > CERNELS_MOE_UP) return 0;
    if (H % 64 || F % 64) return 0;
    return cmoe::packed_weight_bytes(H, F, E, which);
}

int cernels_moe_pack_weights(const void* src, int32_t H, int32_t F, int32_t E, int32_t layout, int32_t which,
                             void* dst, hipStream_t stream) {
    if (!src || !dst || H <= 0 || F <= 0 || E <= 0) return CERNELS_MOE_INVALID_ARGUMENT;
    if (layout != CERNELS_MOE_LAYOUT_CONCAT && layout != CERNELS_MOE_LAYOUT_INTERLEAVED)
        return CERNELS_MOE_INVALID_ARGUMENT;
    if (which < CERNELS_MOE_GATE_UP || which > CERNELS_MOE_UP) return CERNELS_MOE_INVALID_ARGUMENT;
    if (H % 64 || F % 64) return CERNELS_MOE_UNSUPPORTED_SHAPE;
    if (!aligned16(src) || !aligned16(dst)) return CERNELS_MOE_MISALIGNED;
    return hip_status(cmoe::launch_pack(static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), E, H, F,
                                        layout, which, stream));
}

int cernels_moe_experts_packed_staged(const void* x, const void* gate_up_packed, const float* gate_up_bias,
                                      const void* down_packed, const float* down_bias, const int32_t* indices,
                                      const float* weights, int32_t T, int32_t H, int32_t F, int32_t E, int32_t K,
                                      int32_t bias_layout, int32_t act, void* out, void* workspace,
                                      size_t workspace_bytes, hipStream_t stream, hipEvent_t* stage_events) {
    int st = common_checks(x, gate_up_packed, down_packed, indices, weights, T, H, F, E, K, bias_layout, act, out,
                           workspace);
    if (st != CERNELS_MOE_OK || T == 0) return st;
    if (H % 64 || F % 64 || E > kMaxExperts) return CERNELS_MOE_UNSUPPORTED_SHAPE;
    if (!act_gated(act) && gate_up_bias) return CERNELS_MOE_UNSUPPORTED_SHAPE;  // non-gated: no bias
    // The packed GEMMs address x with 32-bit buffer offsets.
    if ((long long)T * H * 2 >= (1LL << 31)) return CERNELS_MOE_UNSUPPORTED_SHAPE;
    const PrefillWs w = prefill_ws(T, H, F, E, K);
    if (workspace_bytes < w.total) return CERNELS_MOE_WORKSPACE_TOO_SMALL;
    char* base = static_cast<char*>(workspace);
    return hip_status(cmoe::launch_prefill_packed(
        x, gate_up_packed, gate_up_bias, down_packed, down_bias, indices, weights, T, H, F, E, K,
        bias_layout == CERNELS_MOE_LAYOUT_INTERLEAVED, act, out, reinterpret_cast<int32_t*>(base + w.offsets),
        reinterpret_cast<int32_t*>(base + w.tile_offsets), reinterpret_cast<int32_t*>(base + w.meta),
        reinterpret_cast<int32_t*>(base + w.sorted_pairs), reinterpret_cast<int32_t*>(base + w.tile_expert),
        reinterpret_cast<int32_t*>(base + w.route_counts), w.capacity, reinterpret_cast<uint16_t*>(base + w.glu),
        reinterpret_cast<float*>(base + w.Y), reinterpret_cast<int8_t*>(base + w.gexp), reinterpret_cast<int8_t*>(base + w.rsig),
        reinterpret_cast<int8_t*>(base + w.psig), stream, stage_events));
}

int cernels_moe_experts_packed(const void* x, const void* gate_up_packed, const float* gate_up_bias,
                               const void* down_packed, const float* down_bias, const int32_t* indices,
                               const float* weights, int32_t T, int32_t H, int32_t F, int32_t E, int32_t K,
                               int32_t bias_layout, int32_t act, void* out, void* workspace, size_t workspace_bytes,
                               hipStream_t stream) {
    return cernels_moe_experts_packed_staged(x, gate_up_packed, gate_up_bias, down_packed, down_bias, indices,
                                             weights, T, H, F, E, K, bias_layout, act, out, workspace,
                                             workspace_bytes, stream, nullptr);
}

// ---- megablocks_moe: non-gated experts on weights as stored, packed into the workspace per call ----

namespace {
static int megablocks_act(int act_id) {
    switch (act_id) {
        case 0: return CERNELS_MOE_ACT_GELU_TANH;
        case 1: return CERNELS_MOE_ACT_SILU_PLAIN;
        case 2: return CERNELS_MOE_ACT_RELU;
        default: return -1;
    }
}
struct MegaWs {
    size_t w1, w2, run, total;
};
static MegaWs megablocks_ws(int T, int H, int F, int E, int K) {
    MegaWs m{};
    m.w1 = 0;
    m.w2 = align_up(cmoe::packed_weight_bytes(H, F, E, CERNELS_MOE_UP));
    m.run = m.w2 + align_up(cmoe::packed_weight_bytes(H, F, E, CERNELS_MOE_DOWN));
    m.total = m.run + prefill_ws(T, H, F, E, K).total;
    return m;
}
}  // namespace

size_t cernels_megablocks_moe_workspace_bytes(int32_t T, int32_t H, int32_t F, int32_t E, int32_t topk) {
    if (!dims_ok(T, H, F, E, topk) || H % 64 || F % 64) return 0;
    return megablocks_ws(T, H, F, E, topk).total;
}

int cernels_megablocks_moe(const void* x, const void* w1, const void* w2, const int32_t* indices, const float* weights,
                           int32_t T, int32_t H, int32_t F, int32_t E, int32_t topk, int32_t act_id, void* out,
                           void* workspace, size_t workspace_bytes, hipStream_t stream) {
    const int act = megablocks_act(act_id);
    if (act < 0) return CERNELS_MOE_INVALID_ARGUMENT;
    int st = common_checks(x, w1, w2, indices, weights, T, H, F, E, topk, CERNELS_MOE_LAYOUT_INTERLEAVED, act, out,
                           workspace);
    if (st != CERNELS_MOE_OK || T == 0) return st;
    if (H % 64 || F % 64 || E > kMaxExperts) return CERNELS_MOE_UNSUPPORTED_SHAPE;
    const MegaWs m = megablocks_ws(T, H, F, E, topk);
    if (workspace_bytes < m.total) return CERNELS_MOE_WORKSPACE_TOO_SMALL;
    char* base = static_cast<char*>(workspace);
    // w1 [E, H, F] and w2 [E, F, H] are both k-major: the interleaved layouts of up and down
    st = cernels_moe_pack_weights(w1, H, F, E, CERNELS_MOE_LAYOUT_INTERLEAVED, CERNELS_MOE_UP, base + m.w1, stream);
    if (st != CERNELS_MOE_OK) return st;
    st = cernels_moe_pack_weights(w2, H, F, E, CERNELS_MOE_LAYOUT_INTERLEAVED, CERNELS_MOE_DOWN, base + m.w2, stream);
    if (st != CERNELS_MOE_OK) return st;
    return cernels_moe_experts_packed(x, base + m.w1, nullptr, base + m.w2, nullptr, indices, weights, T, H, F, E,
                                      topk, CERNELS_MOE_LAYOUT_CONCAT, act, out, base + m.run, workspace_bytes - m.run,
                                      stream);
}

int32_t cernels_moe_decode_max_tokens(void) { return cmoe::decode_max_tokens(); }
int32_t cernels_moe_decode_max_pairs(void) { return cmoe::decode_max_pairs(); }

size_t cernels_moe_experts_decode_workspace_bytes(int32_t T, int32_t H, int32_t F, int32_t E, int32_t K) {
    if (!dims_ok(T, H, F, E, K)) return 0;
    return decode_ws(T, H, F, K).total;
}

namespace {
// Every check of the decode entry except the workspace's size, in the entry's order.
static int decode_checks(const void* x, const void* w1, const void* w2, const int32_t* idx, const float* wts, int T,
                         int H, int F, int E, int K, int layout, int act, void* out, const void* ws) {
    int st = common_checks(x, w1, w2, idx, wts, T, H, F, E, K, layout, act, out, const_cast<void*>(ws));
    if (st != CERNELS_MOE_OK || T == 0) return st;
    if (layout != CERNELS_MOE_LAYOUT_CONCAT || !act_gated(act)) return CERNELS_MOE_UNSUPPORTED_SHAPE;
    if (T > cmoe::decode_max_tokens() || T * K > cmoe::decode_max_pairs()) return CERNELS_MOE_UNSUPPORTED_SHAPE;
    if (H % 8 || F % 8 || E > kMaxExperts || !cmoe::decode_shape_supported(H, F)) return CERNELS_MOE_UNSUPPORTED_SHAPE;
    return CERNELS_MOE_OK;
}
}  // namespace

int cernels_moe_experts_decode_staged(const void* x, const void* gate_up_proj, const float* gate_up_bias,
                                      const void* down_proj, const float* down_bias, const int32_t* indices,
                                      const float* weights, int32_t T, int32_t H, int32_t F, int32_t E, int32_t K,
                                      int32_t layout, int32_t act, void* out, void* workspace,
                                      size_t workspace_bytes, hipStream_t stream, hipEvent_t* stage_events) {
    int st = decode_checks(x, gate_up_proj, down_proj, indices, weights, T, H, F, E, K, layout, act, out, workspace);
    if (st != CERNELS_MOE_OK || T == 0) return st;
    const DecodeWs w = decode_ws(T, H, F, K);
    if (workspace_bytes < w.total) return CERNELS_MOE_WORKSPACE_TOO_SMALL;
    char* base = static_cast<char*>(workspace);
    return hip_status(cmoe::launch_decode(
        static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(gate_up_proj), gate_up_bias,
        static_cast<const uint16_t*>(down_proj), down_bias, indices, weights,
        reinterpret_cast<uint16_t*>(base + w.glu), reinterpret_cast<int32_t*>(base + w.order),
        static_cast<uint16_t*>(out), T, H, F, E, K, act, stream,
        stage_events));
}

int cernels_moe_experts_decode(const void* x, const void* gate_up_proj, const float* gate_up_bias,
                               const void* down_proj, const float* down_bias, const int32_t* indices,
                               const float* weights, int32_t T, int32_t H, int32_t F, int32_t E, int32_t K,
                               int32_t layout, int32_t act, void* out, void* workspace, size_t workspace_bytes,
                               hipStream_t stream) {
    return cernels_moe_experts_decode_staged(x, gate_up_proj, gate_up_bias, down_proj, down_bias, indices, weights,
                                             T, H, F, E, K, layout, act, out, workspace, workspace_bytes, stream,
                                             nullptr);
}

int cernels_moe_experts_decode_noalloc(const void* x, const void* gate_up_proj, const float* gate_up_bias,
                                       const void* down_proj, const float* down_bias, const int32_t* indices,
                                       const float* weights, int32_t T, int32_t H, int32_t F, int32_t E, int32_t K,
                                       int32_t layout, int32_t act, void* out, hipStream_t stream) {
    // The library's static per-GPU scratch takes the place of the workspace. Every check of the decode
    // entry runs first, in its order, so a call is refused exactly as the decode entry refuses it (a
    // shape it accepts always fits the scratch; the size check after them stays as a guard).
    alignas(16) static const unsigned char kStandIn[16] = {};  // the scratch in the pointer checks
    const int st = decode_checks(x, gate_up_proj, down_proj, indices, weights, T, H, F, E, K, layout, act, out,
                                 kStandIn);
    if (st != CERNELS_MOE_OK || T == 0) return st;
    if (decode_ws(T, H, F, K).total > cmoe::decode_noalloc_bytes()) return CERNELS_MOE_WORKSPACE_TOO_SMALL;
    void* ws = nullptr;
    if (cmoe::decode_noalloc_scratch(&ws) != hipSuccess) return CERNELS_MOE_HIP_ERROR;
    return cernels_moe_experts_decode_staged(x, gate_up_proj, gate_up_bias, down_proj, down_bias, indices, weights,
                                             T, H, F, E, K, layout, act, out, ws, cmoe::decode_noalloc_bytes(), stream,
                                             nullptr);
}

// ---- the reference's per-model ops ----------------------------------------------------------------

int cernels_cohere2_moe_experts(const void* x, const void* gate_up_proj, const void* down_proj, const int32_t* indices,
                                const float* weights, int32_t T, int32_t H, int32_t F, int32_t E, int32_t topk,
                                void* out, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    return cernels_moe_experts(x, gate_up_proj, nullptr, down_proj, nullptr, indices, weights, T, H, F, E, topk,
                               CERNELS_MOE_LAYOUT_CONCAT, CERNELS_MOE_ACT_SILU, out, workspace, workspace_bytes,
                               stream);
}

int cernels_cohere2_moe_experts_decode(const void* x, const void* gate_up_proj, const void* down_proj,
                                       const int32_t* indices, const float* weights, int32_t T, int32_t H, int32_t F,
                                       int32_t E, int32_t topk, void* out, void* workspace, size_t workspace_bytes,
                                       hipStream_t stream) {
    return cernels_moe_experts_decode(x, gate_up_proj, nullptr, down_proj, nullptr, indices, weights, T, H, F, E,
                                      topk, CERNELS_MOE_LAYOUT_CONCAT, CERNELS_MOE_ACT_SILU, out, workspace,
                                      workspace_bytes, stream);
}

int cernels_deepseek_ocr2_moe_experts(const void* x, const void* gate_up_proj, const void* down_proj,
                                      const int32_t* indices, const float* weights, int32_t T, int32_t H, int32_t F,
                                      int32_t E, int32_t topk, void* out, void* workspace, size_t workspace_bytes,
                                      hipStream_t stream) {
    return cernels_cohere2_moe_experts(x, gate_up_proj, down_proj, indices, weights, T, H, F, E, topk, out, workspace,
                                       workspace_bytes, stream);
}

int cernels_deepseek_ocr2_moe_experts_decode(const void* x, const void* gate_up_proj, const void* down_proj,
                                             const int32_t* indices, const float* weights, int32_t T, int32_t H,
                                             int32_t F, int32_t E, int32_t topk, void* out, void* workspace,
                                             size_t workspace_bytes, hipStream_t stream) {
    return cernels_cohere2_moe_experts_decode(x, gate_up_proj, down_proj, indices, weights, T, H, F, E, topk, out,
                                              workspace, workspace_bytes, stream);
}

int cernels_qwen3_next_moe_experts(const void* x, const void* gate_up_proj, const void* down_proj,
                                   const int32_t* indices, const float* weights, int32_t T, int32_t H, int32_t F,
                                   int32_t E, int32_t topk, void* out, void* workspace, size_t workspace_bytes,
                                   hipStream_t stream) {
    return cernels_cohere2_moe_experts(x, gate_up_proj, down_proj, indices, weights, T, H, F, E, topk, out, workspace,
                                       workspace_bytes, stream);
}

int cernels_gpt_oss_moe_experts(const void* x, const void* gate_up_proj, const float* gate_up_bias,
                                const void* down_proj, const float* down_bias, const int32_t* indices,
                                const float* weights, int32_t T, int32_t H, int32_t F, int32_t E, int32_t topk,
                                void* out, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    return cernels_moe_experts(x, gate_up_proj, gate_up_bias, down_proj, down_bias, indices, weights, T, H, F, E,
                               topk, CERNELS_MOE_LAYOUT_INTERLEAVED, CERNELS_MOE_ACT_GPTOSS, out, workspace,
                               workspace_bytes, stream);
}

}  // extern "C"
