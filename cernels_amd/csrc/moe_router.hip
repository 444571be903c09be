// Fused MoE router: logits = x Wᵀ (+ b) rounded to bf16, then per-token expert selection, written
// straight in the form the experts op consumes (int32 ids, fp32 weights).
//
// Replaces the routers the reference runs inside its timed gpt-oss and qwen3 ops
// (src/kops/registry/gpt_oss_moe_experts.py:35, src/kops/registry/qwen3_next_moe_experts.py:28),
// i.e. transformers' GptOssTopKRouter (modeling_gpt_oss.py:126-130) and Qwen3NextTopKRouter
// (modeling_qwen3_next.py:766-775): bf16 F.linear, then
//   SOFTMAX_TOPK: probs = softmax_fp32(logits); top-k of probs; optional renormalisation; weights
//                 rounded to bf16 (the logits dtype);
//   TOPK_SOFTMAX: top-k of the logits; softmax over the k values, rounded to bf16.
// Ties (equal values, common with bf16 logits) go to the lower expert id; torch leaves their order
// unspecified. Output weights are the bf16 values widened to fp32, as the loaders' .float() casts.
//
// One workgroup per 32 tokens, 4 waves. The logits GEMM runs on MFMA (32x32x16 bf16, fp32 acc):
// wave w takes the 32-expert column fragments w, w+4, ... four at a time. The bf16-rounded logits
// of the 32 tokens go to LDS; then each wave selects for 8 tokens, a lane holding experts lane,
// lane+64, ... in registers; top-k is k rounds of a wave-wide (value, lowest id) argmax.
#include <type_traits>

#include "moe_common.h"

namespace cmoe {

constexpr int kRtrTokens = 32;
constexpr int kRtrWaves = 4;
constexpr int kRtrThreads = kRtrWaves * kWave;
constexpr int kRtrMaxE = 1024;
constexpr int kRtrMaxK = 32;
constexpr int kRtrFG = 4;  // column fragments per wave pass

constexpr int kRouterSoftmaxTopk = 0;
constexpr int kRouterTopkSoftmax = 1;

__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// Wave-wide argmax: the largest value, ties to the smallest id; every lane returns it.
__device__ __forceinline__ void wave_argmax(float& v, int& id) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, kWave);
        const int oi = __shfl_xor(id, o, kWave);
        if (ov > v || (ov == v && oi < id)) {
            v = ov;
            id = oi;
        }
    }
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

template <int MODE, int EJ>  // EJ = experts per lane = ceil(E / 64)
__global__ __launch_bounds__(kRtrThreads) void moe_router_kernel(const uint16_t* __restrict__ x,
                                                                  const uint16_t* __restrict__ w,
                                                                  const uint16_t* __restrict__ bias, int T, int H,
                                                                  int E, int K, int renorm,
                                                                  int32_t* __restrict__ idx_out,
                                                                  float* __restrict__ w_out,
                                                                  uint16_t* __restrict__ logits_out) {
    __shared__ float s_logit[kRtrTokens][kRtrMaxE];
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int t0 = blockIdx.x * kRtrTokens;
    const int nf = ceil_div(E, 32), ks_n = H / 16;

    // ---- logits on MFMA: lane l feeds token row l % 32 and expert column l % 32, k slot 8 (l / 32)
    const uint16_t* xa = x + (long long)min(t0 + (lane & 31), T - 1) * H + 8 * (lane >> 5);
    for (int fb = wave; fb < nf; fb += kRtrWaves * kRtrFG) {
        const uint16_t* wb[kRtrFG];
#pragma unroll
        for (int g = 0; g < kRtrFG; ++g) {
            const int f = min(fb + g * kRtrWaves, nf - 1);
            wb[g] = w + (long long)min(32 * f + (lane & 31), E - 1) * H + 8 * (lane >> 5);
        }
        f32x16 acc[kRtrFG];
#pragma unroll
        for (int g = 0; g < kRtrFG; ++g)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[g][r] = 0.f;
#pragma unroll 4
        for (int ks = 0; ks < ks_n; ++ks) {
            const bf16x8 a = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(xa + 16 * ks));
#pragma unroll
            for (int g = 0; g < kRtrFG; ++g) {
                const bf16x8 b = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(wb[g] + 16 * ks));
                acc[g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[g], 0, 0, 0);
            }
        }
        // element r of a block: token 8(r/4) + 4(lane/32) + r%4, expert 32 f + lane % 32
#pragma unroll
        for (int g = 0; g < kRtrFG; ++g) {
            const int f = fb + g * kRtrWaves;
            if (f >= nf) break;  // uniform
            const int e = 32 * f + (lane & 31);
            const float be = (bias != nullptr && e < E) ? bf16_bits_to_f32(bias[e]) : 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int tl = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (e < E) s_logit[tl][e] = round_bf16(acc[g][r] + be);
            }
        }
    }
    __syncthreads();

    // ---- per-token selection; wave w takes tokens w, w+4, ...
    for (int tl = wave; tl < kRtrTokens; tl += kRtrWaves) {
        const int t = t0 + tl;
        if (t >= T) break;  // uniform
        float v[EJ];
#pragma unroll
        for (int j = 0; j < EJ; ++j) {
            const int e = lane + kWave * j;
            v[j] = e < E ? s_logit[tl][e] : -INFINITY;
            if (logits_out != nullptr && e < E) logits_out[(long long)t * E + e] = f32_to_bf16_bits(v[j]);
        }
        if constexpr (MODE == kRouterSoftmaxTopk) {
            float m = -INFINITY;
#pragma unroll
            for (int j = 0; j < EJ; ++j) m = fmaxf(m, v[j]);
            m = wave_max(m);
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < EJ; ++j) {
                v[j] = lane + kWave * j < E ? __expf(v[j] - m) : 0.f;
                s += v[j];
            }
            s = wave_sum(s);
#pragma unroll
            for (int j = 0; j < EJ; ++j) v[j] = lane + kWave * j < E ? v[j] / s : -INFINITY;
        }
        // top-k: k rounds of a wave-wide argmax; the winner is removed from its lane
        float sel_v = 0.f;  // lane k keeps the k-th value and id
        int sel_i = 0;
        float top_first = 0.f, sum_sel = 0.f;
        for (int k = 0; k < K; ++k) {
            float bv = -INFINITY;
            int bi = 0x7fffffff;
#pragma unroll
            for (int j = 0; j < EJ; ++j) {
                const int e = lane + kWave * j;
                if (v[j] > bv || (v[j] == bv && e < bi)) {
                    bv = v[j];
                    bi = e;
                }
            }
            wave_argmax(bv, bi);
#pragma unroll
            for (int j = 0; j < EJ; ++j)
                if (lane + kWave * j == bi) v[j] = -INFINITY;
            if (lane == k) {
                sel_v = bv;
                sel_i = bi;
            }
            if (k == 0) top_first = bv;
            sum_sel += MODE == kRouterSoftmaxTopk ? bv : 0.f;
        }
        float wt;
        if constexpr (MODE == kRouterSoftmaxTopk) {
            wt = renorm ? sel_v / sum_sel : sel_v;
        } else {
            // softmax over the k selected logits; top_first is their maximum
            const float ex = lane < K ? __expf(sel_v - top_first) : 0.f;
            wt = ex / wave_sum(ex);
        }
        if (lane < K) {
            idx_out[(long long)t * K + lane] = sel_i;
            w_out[(long long)t * K + lane] = round_bf16(wt);
        }
    }
}

int router_max_experts() { return kRtrMaxE; }
int router_max_topk() { return kRtrMaxK; }

template <int MODE>
static hipError_t launch_router_m(const uint16_t* x, const uint16_t* w, const uint16_t* bias, int T, int H, int E,
                                  int K, int renorm, int32_t* idx, float* wt, uint16_t* logits, hipStream_t s) {
    const dim3 grid(ceil_div(T, kRtrTokens));
    const int ej = ceil_div(E, kWave);
#define CMOE_RTR(EJ) \
    hipLaunchKernelGGL((moe_router_kernel<MODE, EJ>), grid, dim3(kRtrThreads), 0, s, x, w, bias, T, H, E, K, renorm, \
                       idx, wt, logits)
    if (ej <= 1) CMOE_RTR(1);
    else if (ej <= 2) CMOE_RTR(2);
    else if (ej <= 4) CMOE_RTR(4);
    else if (ej <= 8) CMOE_RTR(8);
    else CMOE_RTR(16);
#undef CMOE_RTR
    return hipGetLastError();
}

// Shapes were checked by the caller: 1 <= K <= min(E, 32), E <= 1024, H % 16 == 0, T >= 1.
hipError_t launch_router(const uint16_t* x, const uint16_t* w, const uint16_t* bias, int T, int H, int E, int K,
                         int mode, int renorm, int32_t* idx, float* wt, uint16_t* logits, hipStream_t s) {
    if (mode == kRouterSoftmaxTopk) return launch_router_m<kRouterSoftmaxTopk>(x, w, bias, T, H, E, K, renorm, idx, wt, logits, s);
    return launch_router_m<kRouterTopkSoftmax>(x, w, bias, T, H, E, K, renorm, idx, wt, logits, s);
}

}  // namespace cmoe
