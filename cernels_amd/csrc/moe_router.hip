// Fused MoE router: logits = x Wᵀ (+ b) rounded to bf16, then per-token expert selection, written
// straight in the form the experts op consumes (int32 ids, fp32 weights), plus the bf16 logits.
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
// The logits GEMM ([T,H] x [E,H]ᵀ) runs on MFMA (32x32x16 bf16, fp32 accumulation) from LDS: each
// stage holds 64 k-columns of the token rows and expert rows, copied HBM -> LDS directly
// (global_load_lds_dwordx4, eight lanes per 128-byte row segment) into a ring of stages with several
// in flight, one wait and one barrier per stage.
//   E <= 64  (gpt-oss): one kernel. A workgroup owns 32 tokens and all experts; its four waves
//            split each stage's four k-steps, their partial sums meet in LDS (fixed order), and
//            the same workgroup selects for its 32 tokens.
//   E > 64   (qwen3-next): a 128-token x 64-expert tiled GEMM writes the bf16 logits, then a
//            selection kernel (one wave per token) reads them back.
// Selection: a lane holds experts lane, lane+64, ...; each expert becomes a 32-bit key (logit
// order, then lower id) and top-k is k rounds of a DPP wave maximum over the lanes' sorted heads.
#include <type_traits>

#include "moe_common.h"
#include "moe_tile.h"

namespace cmoe {

constexpr int kRtrThreads = 256;  // 4 waves
constexpr int kRtrMaxE = 1024;
constexpr int kRtrMaxK = 32;
constexpr int kRtrFusedMaxE = 64;

constexpr int kRouterSoftmaxTopk = 0;
constexpr int kRouterTopkSoftmax = 1;

__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// ---- wave reductions over DPP: row_shr 1, 2, 4, 8 within rows of 16 lanes, then row_bcast 15 and
// 31 carry row results up; lane 63 ends with the reduction of all 64 lanes, read back as a uniform
// value. Lanes a DPP source does not reach contribute 0, the identity of both reductions below.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_or_zero(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, false);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_or_zero<0x111, 0xf>(v));
    v = max(v, dpp_or_zero<0x112, 0xf>(v));
    v = max(v, dpp_or_zero<0x114, 0xf>(v));
    v = max(v, dpp_or_zero<0x118, 0xf>(v));
    v = max(v, dpp_or_zero<0x142, 0xa>(v));
    v = max(v, dpp_or_zero<0x143, 0xc>(v));
    return __builtin_amdgcn_readlane(v, 63);
}

__device__ __forceinline__ float wave_sum_f32(float v) {
    v += __uint_as_float(dpp_or_zero<0x111, 0xf>(__float_as_uint(v)));
    v += __uint_as_float(dpp_or_zero<0x112, 0xf>(__float_as_uint(v)));
    v += __uint_as_float(dpp_or_zero<0x114, 0xf>(__float_as_uint(v)));
    v += __uint_as_float(dpp_or_zero<0x118, 0xf>(__float_as_uint(v)));
    v += __uint_as_float(dpp_or_zero<0x142, 0xa>(__float_as_uint(v)));
    v += __uint_as_float(dpp_or_zero<0x143, 0xc>(__float_as_uint(v)));
    return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 63));
}

// Selection key: the bf16 logit mapped to an order-preserving 16-bit code (larger logit, larger
// code; -0 ranks as +0) in the high half, 0xffff - expert id in the low half, so that one unsigned
// max picks the largest logit and, among equal logits, the lowest id. Every real key is nonzero
// (the code of -inf is 0x007f); 0 marks "none".
__device__ __forceinline__ uint32_t order_key(float logit, int e) {
    uint32_t b = __float_as_uint(logit) >> 16;  // the logit is a bf16 value
    if (b == 0x8000u) b = 0u;
    const uint32_t o = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
    return (o << 16) | (0xffffu - (uint32_t)e);
}
__device__ __forceinline__ float key_logit(uint32_t key) {
    const uint32_t o = key >> 16;
    return __uint_as_float(((o & 0x8000u) ? (o & 0x7fffu) : (~o & 0xffffu)) << 16);
}
__device__ __forceinline__ int key_expert(uint32_t key) { return (int)(0xffffu - (key & 0xffffu)); }

// Bitonic sort of N (a power of two) keys into descending order, in registers.
template <int N>
__device__ __forceinline__ void sort_desc(uint32_t (&a)[N]) {
#pragma unroll
    for (int k = 2; k <= N; k <<= 1)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1)
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const int l = i ^ j;
                if (l > i) {
                    const uint32_t hi = max(a[i], a[l]), lo = min(a[i], a[l]);
                    const bool desc = (i & k) == 0;
                    a[i] = desc ? hi : lo;
                    a[l] = desc ? lo : hi;
                }
            }
}

// Selection for token t by one wave (all 64 lanes active). v[j] = bf16 logit of expert lane + 64 j.
// Output row t has K + S slots: the K chosen experts, then S shared-expert slots with ids E..E+S-1
// and weight bf16(sigmoid(gate_logit)) (the Qwen3-Next shared-expert gate, modeling_qwen3_next.py:794).
// The experts are chosen on the logits in both modes: softmax is strictly increasing, so the top-k
// of the probabilities is the top-k of the logits, and equal probabilities come only from equal
// logits. Each lane sorts its keys; round k takes the wave-wide maximum of the lanes' heads and the
// lane holding it pops its head. Lane k keeps the k-th key.
template <int MODE, int EJ>
__device__ __forceinline__ void select_token(const float (&v)[EJ], int lane, long long t, int E, int K, int renorm,
                                             int S, float gate_logit, int32_t* __restrict__ idx_out,
                                             float* __restrict__ w_out) {
    uint32_t key[EJ];
#pragma unroll
    for (int j = 0; j < EJ; ++j) key[j] = lane + kWave * j < E ? order_key(v[j], lane + kWave * j) : 0u;
    sort_desc<EJ>(key);
    uint32_t sel = 0u, top = 0u;
    for (int k = 0; k < K; ++k) {
        const uint32_t best = wave_max_u32(key[0]);
        if (k == 0) top = best;
        if (lane == k) sel = best;
        const bool pop = key[0] == best;
#pragma unroll
        for (int j = 0; j + 1 < EJ; ++j) key[j] = pop ? key[j + 1] : key[j];
        key[EJ - 1] = pop ? 0u : key[EJ - 1];
    }
    const float lmax = key_logit(top), lsel = key_logit(sel);
    float wt;
    if constexpr (MODE == kRouterSoftmaxTopk) {
        // p = exp(l - max) / sum over all experts of exp(l_j - max), the fp32 softmax
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < EJ; ++j) s += lane + kWave * j < E ? __expf(v[j] - lmax) : 0.f;
        s = wave_sum_f32(s);
        const float p = lane < K ? __expf(lsel - lmax) / s : 0.f;
        wt = renorm ? p / wave_sum_f32(p) : p;
    } else {
        // softmax over the k selected logits; lmax is their maximum
        const float ex = lane < K ? __expf(lsel - lmax) : 0.f;
        wt = ex / wave_sum_f32(ex);
    }
    const int KO = K + S;
    if (lane < K) {
        idx_out[t * KO + lane] = key_expert(sel);
        w_out[t * KO + lane] = round_bf16(wt);
    } else if (lane < KO) {
        idx_out[t * KO + lane] = E + lane - K;
        w_out[t * KO + lane] = round_bf16(1.f / (1.f + __expf(-gate_logit)));
    }
}

// Stage ring: a stage holds 64 k-columns of ROWS rows = tokens t0.. (rows [0, TM)) then experts
// e0.. (rows [TM, ROWS)), as 128-byte rows in the swizzled layout of lds_off. The copies go straight
// from HBM to LDS (global_load_lds_dwordx4): instruction i of a stage fills rows 8i..8i+7, lane l
// taking row 8i + l/8 and the chunk that the swizzle puts at position l % 8. Wave w issues
// instructions w, w+4, ... (ROWS / 32 each). Rows beyond T or E are clamped (their results are
// never stored); columns beyond H are clamped to H - 8 (their k-steps are skipped), so every
// address is inside x or W.
template <int ROWS, int TM>
struct StageRing {
    static constexpr int kStageBytes = ROWS * kBK * 2;
    static constexpr int kPerWave = ROWS / 32;
    static_assert(ROWS % 32 == 0, "four waves issue whole 8-row instructions");

    __device__ __forceinline__ static void issue(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                 int t0, int e0, int T, int E, int H, int st, uint32_t slot,
                                                 int wave, int lane) {
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int i = wave + 4 * j;
            const int row = 8 * i + (lane >> 3);
            const int chunk = (lane & 7) ^ swz(row);
            const int k = min(st * kBK + 8 * chunk, H - 8);
            const uint16_t* src = row < TM ? x + (long long)min(t0 + row, T - 1) * H
                                           : w + (long long)min(e0 + row - TM, E - 1) * H;
            dma16(src + k, slot + 1024u * i);
        }
    }
};

// Fragment of rows row0..row0+31 for k-step q of a stage: lane l reads row l % 32, 8 bf16 at
// k = 16 q + 8 (l / 32).
__device__ __forceinline__ bf16x8 lds_frag(const char* __restrict__ stage, int row0, int q, int lane) {
    return __builtin_bit_cast(bf16x8,
                              *reinterpret_cast<const u32x4*>(stage + lds_off(row0 + (lane & 31), 2 * q + (lane >> 5))));
}

// Stage pipeline shared by both GEMMs: S-1 stages in flight; per stage one wait on this wave's own
// copies, one barrier that publishes the stage (and frees the slot read one stage earlier), then the
// copy of stage st + S - 1 into that slot, then compute(stage pointer, st).
template <int S, int ROWS, int TM, typename Compute>
__device__ __forceinline__ void stage_pipeline(char* ring, const uint16_t* __restrict__ x,
                                               const uint16_t* __restrict__ w, int t0, int e0, int T, int E, int H,
                                               int wave, int lane, Compute&& compute) {
    using R = StageRing<ROWS, TM>;
    const int nst = ceil_div(H, kBK);
    const uint32_t base = lds_u32(ring);
#pragma unroll
    for (int s = 0; s < S - 1; ++s)
        if (s < nst) R::issue(x, w, t0, e0, T, E, H, s, base + s * R::kStageBytes, wave, lane);
    for (int st = 0; st < nst; ++st) {
        if (st + S - 2 < nst) wait_vmcnt<(S - 2) * R::kPerWave>();  // stages st+1 .. st+S-2 may stay in flight
        else wait_vmcnt<0>();
        __syncthreads();
        const int nx = st + S - 1;
        if (nx < nst) R::issue(x, w, t0, e0, T, E, H, nx, base + (nx % S) * R::kStageBytes, wave, lane);
        compute(ring + (st % S) * R::kStageBytes, st);
    }
    __syncthreads();
}

// ---- E <= 64: GEMM + selection in one kernel; grid = ceil(T / 32)
constexpr int kRtrFusedStages = 8;
template <int MODE, int NT>  // NT = expert blocks of 32 (1 or 2)
__global__ __launch_bounds__(kRtrThreads) void moe_router_fused_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const uint16_t* __restrict__ bias, int T, int H,
    int E, int K, int renorm, int S, int32_t* __restrict__ idx_out, float* __restrict__ w_out,
    uint16_t* __restrict__ logits_out) {
    constexpr int TM = 32, EN = 32 * NT, ROWS = TM + EN;
    const int ER = E + (S > 0);  // rows of W and of a logits row: the experts, then the shared-expert gate
    constexpr int kRing = kRtrFusedStages * ROWS * kBK * 2;
    static_assert(4 * TM * EN * 4 <= kRing, "partial sums reuse the stage ring");
    __shared__ __align__(1024) char ring[kRing];
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int t0 = blockIdx.x * TM;

    f32x16 acc[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[n][r] = 0.f;
    // wave q takes k-step q of every stage; a k-step at or beyond H is skipped
    stage_pipeline<kRtrFusedStages, ROWS, TM>(ring, x, w, t0, 0, T, ER, H, wave, lane, [&](const char* sb, int st) {
        if (st * kBK + 16 * wave < H) {
            const bf16x8 a = lds_frag(sb, 0, wave, lane);
#pragma unroll
            for (int n = 0; n < NT; ++n)
                acc[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, lds_frag(sb, TM + 32 * n, wave, lane), acc[n], 0, 0, 0);
        }
    });
    // partial sums of the four waves: element r is token 8(r/4) + 4(lane/32) + r%4, expert 32 n + lane % 32
    float(*part)[TM][EN] = reinterpret_cast<float(*)[TM][EN]>(ring);
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int r = 0; r < 16; ++r) part[wave][8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)][32 * n + (lane & 31)] = acc[n][r];
    __syncthreads();
    // logit = bf16(((p0 + p1) + p2) + p3 + b); kept in slice 0 and written to logits_out
    for (int c = tid; c < TM * EN; c += kRtrThreads) {
        const int tl = c / EN, e = c % EN;
        if (e >= ER) continue;
        const float b = bias != nullptr ? bf16_bits_to_f32(bias[e]) : 0.f;
        const float v = round_bf16(((part[0][tl][e] + part[1][tl][e]) + part[2][tl][e]) + part[3][tl][e] + b);
        part[0][tl][e] = v;
        if (t0 + tl < T) logits_out[(long long)(t0 + tl) * ER + e] = f32_to_bf16_bits(v);
    }
    __syncthreads();
    for (int tl = wave; tl < TM; tl += 4) {
        if (t0 + tl >= T) break;  // uniform
        float v[1] = {lane < E ? part[0][tl][lane] : -INFINITY};
        select_token<MODE, 1>(v, lane, t0 + tl, E, K, renorm, S, S > 0 ? part[0][tl][E] : 0.f, idx_out, w_out);
    }
}

// ---- E > 64: tiled logits GEMM, 128 tokens x 64 experts per workgroup; grid = (ceil(T/128), ceil(E/64));
// logits rows are ldl apart (E + 1 with a shared-expert gate, whose logit the selection kernel adds)
constexpr int kRtrTiledStages = 4;
__global__ __launch_bounds__(kRtrThreads) void moe_router_logits_kernel(const uint16_t* __restrict__ x,
                                                                        const uint16_t* __restrict__ w,
                                                                        const uint16_t* __restrict__ bias, int T,
                                                                        int H, int E, int ldl,
                                                                        uint16_t* __restrict__ logits_out) {
    constexpr int TM = 128, EN = 64, ROWS = TM + EN;
    __shared__ __align__(1024) char ring[kRtrTiledStages * ROWS * kBK * 2];
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int t0 = blockIdx.x * TM, e0 = blockIdx.y * EN;

    f32x16 acc[2];
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[n][r] = 0.f;
    // wave w owns token rows 32w..32w+31 and both expert blocks
    stage_pipeline<kRtrTiledStages, ROWS, TM>(ring, x, w, t0, e0, T, E, H, wave, lane, [&](const char* sb, int st) {
        if (st * kBK + kBK <= H) {
#pragma unroll
            for (int q = 0; q < kBK / 16; ++q) {
                const bf16x8 a = lds_frag(sb, 32 * wave, q, lane);
#pragma unroll
                for (int n = 0; n < 2; ++n)
                    acc[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, lds_frag(sb, TM + 32 * n, q, lane), acc[n], 0, 0, 0);
            }
        } else {
            for (int q = 0; st * kBK + 16 * q < H; ++q) {  // last stage of an H that is not a multiple of 64
                const bf16x8 a = lds_frag(sb, 32 * wave, q, lane);
#pragma unroll
                for (int n = 0; n < 2; ++n)
                    acc[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, lds_frag(sb, TM + 32 * n, q, lane), acc[n], 0, 0, 0);
            }
        }
    });
#pragma unroll
    for (int n = 0; n < 2; ++n) {
        const int e = e0 + 32 * n + (lane & 31);
        if (e >= E) continue;
        const float b = bias != nullptr ? bf16_bits_to_f32(bias[e]) : 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = t0 + 32 * wave + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (t < T) logits_out[(long long)t * ldl + e] = f32_to_bf16_bits(acc[n][r] + b);
        }
    }
}

// ---- E > 64: selection from the bf16 logits, one wave per token; grid = ceil(T / 4)
// With S > 0 the wave also computes the shared-expert gate logit, bf16(x_t . w_E (+ b_E)), as a dot
// product over H (16 bf16 per lane per step, fp32, DPP sum) and stores it in logits column E.
template <int MODE, int EJ>  // EJ = experts per lane = ceil(E / 64)
__global__ __launch_bounds__(kRtrThreads) void moe_router_select_kernel(
    uint16_t* __restrict__ logits, const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ bias, int T, int H, int E, int K, int renorm, int S, int32_t* __restrict__ idx_out,
    float* __restrict__ w_out) {
    const int lane = threadIdx.x & (kWave - 1);
    const int t = blockIdx.x * 4 + (int)(threadIdx.x / kWave);
    if (t >= T) return;  // uniform per wave
    uint16_t* row = logits + (long long)t * (E + (S > 0));
    float gate = 0.f;
    if (S > 0) {
        const uint16_t* xr = x + (long long)t * H;
        const uint16_t* gr = w + (long long)E * H;
        float acc = 0.f;
        for (int h = 8 * lane; h < H; h += 8 * kWave) {  // H % 16 == 0: whole 8-element chunks
            const u32x4 xa = *reinterpret_cast<const u32x4*>(xr + h);
            const u32x4 ga = *reinterpret_cast<const u32x4*>(gr + h);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc = fmaf(__uint_as_float(xa[q] << 16), __uint_as_float(ga[q] << 16), acc);
                acc = fmaf(__uint_as_float(xa[q] & 0xffff0000u), __uint_as_float(ga[q] & 0xffff0000u), acc);
            }
        }
        gate = round_bf16(wave_sum_f32(acc) + (bias != nullptr ? bf16_bits_to_f32(bias[E]) : 0.f));
        if (lane == 0) row[E] = f32_to_bf16_bits(gate);
    }
    float v[EJ];
#pragma unroll
    for (int j = 0; j < EJ; ++j) {
        const int e = lane + kWave * j;
        v[j] = e < E ? bf16_bits_to_f32(row[e]) : -INFINITY;
    }
    select_token<MODE, EJ>(v, lane, t, E, K, renorm, S, gate, idx_out, w_out);
}

int router_max_experts() { return kRtrMaxE; }
int router_max_topk() { return kRtrMaxK; }

template <int MODE>
static hipError_t launch_router_m(const uint16_t* x, const uint16_t* w, const uint16_t* bias, int T, int H, int E,
                                  int K, int renorm, int S, int32_t* idx, float* wt, uint16_t* logits, hipStream_t s) {
    const int ER = E + (S > 0);
    if (ER <= kRtrFusedMaxE) {
        const dim3 grid(ceil_div(T, 32));
        if (ER <= 32)
            hipLaunchKernelGGL((moe_router_fused_kernel<MODE, 1>), grid, dim3(kRtrThreads), 0, s, x, w, bias, T, H, E,
                               K, renorm, S, idx, wt, logits);
        else
            hipLaunchKernelGGL((moe_router_fused_kernel<MODE, 2>), grid, dim3(kRtrThreads), 0, s, x, w, bias, T, H, E,
                               K, renorm, S, idx, wt, logits);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(moe_router_logits_kernel, dim3(ceil_div(T, 128), ceil_div(E, 64)), dim3(kRtrThreads), 0, s,
                       x, w, bias, T, H, E, ER, logits);
    const dim3 grid(ceil_div(T, 4));
    const int ej = ceil_div(E, kWave);
#define CMOE_RTR(EJ) \
    hipLaunchKernelGGL((moe_router_select_kernel<MODE, EJ>), grid, dim3(kRtrThreads), 0, s, logits, x, w, bias, T, H, \
                       E, K, renorm, S, idx, wt)
    if (ej <= 2) CMOE_RTR(2);
    else if (ej <= 4) CMOE_RTR(4);
    else if (ej <= 8) CMOE_RTR(8);
    else CMOE_RTR(16);
#undef CMOE_RTR
    return hipGetLastError();
}

// Shapes were checked by the caller: 1 <= K <= min(E, 32), 0 <= S <= 32, E + (S > 0) <= 1024,
// H % 16 == 0, T >= 1; W and bias have E + (S > 0) rows, logits is [T, E + (S > 0)] bf16, ids and
// weights are [T, K + S].
hipError_t launch_router(const uint16_t* x, const uint16_t* w, const uint16_t* bias, int T, int H, int E, int K,
                         int mode, int renorm, int S, int32_t* idx, float* wt, uint16_t* logits, hipStream_t s) {
    if (mode == kRouterSoftmaxTopk)
        return launch_router_m<kRouterSoftmaxTopk>(x, w, bias, T, H, E, K, renorm, S, idx, wt, logits, s);
    return launch_router_m<kRouterTopkSoftmax>(x, w, bias, T, H, E, K, renorm, S, idx, wt, logits, s);
}

}  // namespace cmoe
