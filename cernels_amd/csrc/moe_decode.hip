// Decode path (few tokens): fused gather-GEMV over the selected experts only.
//
// Replaces decode_gateup_swiglu_kernel / decode_down_accum_kernel + zeros + cast
// (src/kops/cohere2_moe_experts/csrc/cohere2_moe_experts.cu:135-236). Differences by design:
//   * work is split by DISTINCT expert, so an expert picked by several (token, slot) pairs
//     streams its weights from HBM once (the reference streams them once per pair, .cu:143,179);
//   * 64-lane waves read 16-byte chunks of a weight row (1 KB per wave instruction);
//   * the top-k combine is fused into the down GEMV: a workgroup owns whole output rows and sums
//     every (expert, pair) contribution for them in a fixed order, then writes bf16 — no fp32
//     atomics, no cross-workgroup synchronisation, no zero-fill or cast kernel. Two launches.
//
// Layout: concat only (gate_up [E, 2F, H], down [E, H, F]); the reference has no decode entry
// for the interleaved gpt-oss layout either.
//
// Each workgroup rebuilds the routing plan for the <= 256 pairs in LDS: the distinct experts in
// ascending order and, per expert, its pairs in (slot, token) order.
#include "moe_common.h"

namespace cmoe {

constexpr int kDecThreads = 256;
constexpr int kDecWaves = kDecThreads / kWave;
constexpr int kDecMaxPairs = 256;
constexpr int kDecMaxTokens = 64;
constexpr int kDecRowsPerWaveG = 2;   // gate_up kernel: F rows per wave (each = a gate and an up row)
constexpr int kDecRowsPerWaveD = 4;   // down kernel: H rows per workgroup (every wave holds all 4)
constexpr int kDecFBlock = kDecWaves * kDecRowsPerWaveG;  // 8

struct DecodePlan {
    int e[kDecMaxPairs];       // expert of pair p, -1 if out of range
    int spair[kDecMaxPairs];   // pairs in (expert, slot, token) order
    int dexp[kDecMaxPairs];    // distinct experts, ascending
    int dstart[kDecMaxPairs + 1];
    int first[kDecMaxPairs];
    int U;
};

__device__ void build_plan(DecodePlan& pl, const int32_t* __restrict__ idx, int T, int K, int E) {
    const int P = T * K, tid = threadIdx.x;
    for (int p = tid; p < P; p += kDecThreads) {
        const int v = idx[p];
        pl.e[p] = ((unsigned)v < (unsigned)E) ? v : -1;
    }
    __syncthreads();
    int less = 0;
    const int p = tid;  // P <= kDecThreads is checked on the host
    const int ep = p < P ? pl.e[p] : -1;
    if (ep >= 0) {
        const int key = (p % K) * T + p / K;
        int same_before = 0;
        for (int q = 0; q < P; ++q) {
            const int eq = pl.e[q];
            if (eq < 0) continue;
            if (eq < ep) ++less;
            else if (eq == ep && (q % K) * T + q / K < key) ++same_before;
        }
        pl.spair[less + same_before] = p;
        pl.first[p] = same_before == 0;
    } else if (p < P) {
        pl.first[p] = 0;
    }
    const int nvalid = __syncthreads_count(ep >= 0);
    const int U = __syncthreads_count(p < P && pl.first[p]);
    if (p < P && pl.first[p]) {
        int u = 0;
        for (int q = 0; q < P; ++q) u += (pl.first[q] && pl.e[q] < ep);
        pl.dexp[u] = ep;
        pl.dstart[u] = less;
    }
    if (tid == 0) {
        pl.dstart[U] = nvalid;
        pl.U = U;
    }
    __syncthreads();
}

template <int MAXC>
__device__ __forceinline__ void load_row(const uint16_t* __restrict__ row, int nch, int lane, u32x4 (&v)[MAXC]) {
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
        const int c = lane + kWave * i;
        if (c < nch) v[i] = *reinterpret_cast<const u32x4*>(row + 8 * c);
        else v[i] = u32x4{0u, 0u, 0u, 0u};
    }
}

__device__ __forceinline__ float dot8_bf16(const u32x4& a, const u32x4& b, float acc) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        acc = fmaf(bf16_lo(a[d]), bf16_lo(b[d]), acc);
        acc = fmaf(bf16_hi(a[d]), bf16_hi(b[d]), acc);
    }
    return acc;
}

__device__ __forceinline__ float dot8_bf16_f32(const u32x4& w, const f32x4& g0, const f32x4& g1, float acc) {
    acc = fmaf(bf16_lo(w[0]), g0[0], acc);
    acc = fmaf(bf16_hi(w[0]), g0[1], acc);
    acc = fmaf(bf16_lo(w[1]), g0[2], acc);
    acc = fmaf(bf16_hi(w[1]), g0[3], acc);
    acc = fmaf(bf16_lo(w[2]), g1[0], acc);
    acc = fmaf(bf16_hi(w[2]), g1[1], acc);
    acc = fmaf(bf16_lo(w[3]), g1[2], acc);
    acc = fmaf(bf16_hi(w[3]), g1[3], acc);
    return acc;
}

// glu[p, f] = bf16(act(x[t] . W1_e[f] + b, x[t] . W1_e[F+f] + b)) for every pair p of expert e.
// grid: (ceil(F / 8), P); blockIdx.y = distinct-expert slot. Each wave owns 2 consecutive f and
// keeps their 4 weight rows (2 gate + 2 up) in flight at once.
template <int ACT, bool HAS_BIAS, int MAXC>
__global__ __launch_bounds__(kDecThreads) void moe_decode_gateup_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1, const float* __restrict__ b1,
    const int32_t* __restrict__ idx, uint16_t* __restrict__ glu, int T, int H, int F, int E, int K) {
    __shared__ DecodePlan pl;
    build_plan(pl, idx, T, K, E);
    const int u = blockIdx.y;
    if (u >= pl.U) return;
    const int e = pl.dexp[u], ps = pl.dstart[u], pe = pl.dstart[u + 1];
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int nch = H / 8;
    const uint16_t* we = w1 + (long long)e * 2 * F * H;
    const int f0 = blockIdx.x * kDecFBlock + wave * kDecRowsPerWaveG;
    if (f0 >= F) return;
    const int f1 = min(f0 + 1, F - 1);
    u32x4 wg0[MAXC], wu0[MAXC], wg1[MAXC], wu1[MAXC];
    load_row<MAXC>(we + (long long)f0 * H, nch, lane, wg0);
    load_row<MAXC>(we + (long long)(F + f0) * H, nch, lane, wu0);
    load_row<MAXC>(we + (long long)f1 * H, nch, lane, wg1);
    load_row<MAXC>(we + (long long)(F + f1) * H, nch, lane, wu1);
    float bg0 = 0.f, bu0 = 0.f, bg1 = 0.f, bu1 = 0.f;
    if constexpr (HAS_BIAS) {
        const float* be = b1 + (long long)e * 2 * F;
        bg0 = be[f0], bu0 = be[F + f0], bg1 = be[f1], bu1 = be[F + f1];
    }
    for (int s = ps; s < pe; ++s) {
        const int p = pl.spair[s];
        const int t = p / K;
        u32x4 xv[MAXC];
        load_row<MAXC>(x + (long long)t * H, nch, lane, xv);
        float g0 = 0.f, u0 = 0.f, g1 = 0.f, u1 = 0.f;
#pragma unroll
        for (int i = 0; i < MAXC; ++i) {
            g0 = dot8_bf16(wg0[i], xv[i], g0);
            u0 = dot8_bf16(wu0[i], xv[i], u0);
            g1 = dot8_bf16(wg1[i], xv[i], g1);
            u1 = dot8_bf16(wu1[i], xv[i], u1);
        }
        g0 = wave_sum(g0);
        u0 = wave_sum(u0);
        g1 = wave_sum(g1);
        u1 = wave_sum(u1);
        if (lane == 0) glu[(long long)p * F + f0] = f32_to_bf16_bits(swiglu<ACT>(g0 + bg0, u0 + bu0));
        if (lane == 1 && f0 + 1 < F) glu[(long long)p * F + f0 + 1] = f32_to_bf16_bits(swiglu<ACT>(g1 + bg1, u1 + bu1));
    }
}

// out[t, h] = bf16( sum over pairs (t,k) of w_p * (glu[p] . W2_e[h] + b2_e[h]) ).
// grid: ceil(H / 4). A workgroup owns 4 output rows for every token; its 4 waves split the
// distinct experts (wave w takes experts w, w+4, ...), each wave holding the 4 weight rows of an
// expert in registers and reusing every glu chunk for all 4 rows. Per-wave partial sums meet in
// LDS and are added in wave order, so the result does not depend on timing.
template <bool HAS_BIAS, int MAXC>
__global__ __launch_bounds__(kDecThreads) void moe_decode_down_kernel(
    const uint16_t* __restrict__ glu, const uint16_t* __restrict__ w2, const float* __restrict__ b2,
    const int32_t* __restrict__ idx, const float* __restrict__ route_w, uint16_t* __restrict__ out, int T, int H,
    int F, int E, int K) {
    __shared__ DecodePlan pl;
    __shared__ float part[kDecWaves][kDecRowsPerWaveD][kDecMaxTokens];
    build_plan(pl, idx, T, K, E);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int h0 = blockIdx.x * kDecRowsPerWaveD;
    const int nch = F / 8;
    float acc[kDecRowsPerWaveD];
#pragma unroll
    for (int j = 0; j < kDecRowsPerWaveD; ++j) acc[j] = 0.f;  // lane t holds token t's partial sums

    for (int u = wave; u < pl.U; u += kDecWaves) {
        const int e = pl.dexp[u], ps = pl.dstart[u], pe = pl.dstart[u + 1];
        const uint16_t* we = w2 + (long long)e * H * F;
        u32x4 wr[kDecRowsPerWaveD][MAXC];
#pragma unroll
        for (int j = 0; j < kDecRowsPerWaveD; ++j)
            load_row<MAXC>(we + (long long)min(h0 + j, H - 1) * F, nch, lane, wr[j]);
        float bj[kDecRowsPerWaveD];
#pragma unroll
        for (int j = 0; j < kDecRowsPerWaveD; ++j) {
            bj[j] = 0.f;
            if constexpr (HAS_BIAS) bj[j] = b2[(long long)e * H + min(h0 + j, H - 1)];
        }
        for (int s = ps; s < pe; ++s) {
            const int p = pl.spair[s];
            u32x4 gv[MAXC];
            load_row<MAXC>(glu + (long long)p * F, nch, lane, gv);
            float d[kDecRowsPerWaveD];
#pragma unroll
            for (int j = 0; j < kDecRowsPerWaveD; ++j) {
                d[j] = 0.f;
#pragma unroll
                for (int i = 0; i < MAXC; ++i) d[j] = dot8_bf16(wr[j][i], gv[i], d[j]);
            }
            const float wp = route_w[p];
            const int t = p / K;
#pragma unroll
            for (int j = 0; j < kDecRowsPerWaveD; ++j) {
                const float v = wave_sum(d[j]);
                if (lane == t) acc[j] += wp * (v + bj[j]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < kDecRowsPerWaveD; ++j) part[wave][j][lane] = acc[j];
    __syncthreads();
    for (int i = threadIdx.x; i < kDecRowsPerWaveD * T; i += kDecThreads) {
        const int j = i / T, t = i - j * T, h = h0 + j;
        if (h >= H) continue;
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < kDecWaves; ++w) sum += part[w][j][t];
        out[(long long)t * H + h] = f32_to_bf16_bits(sum);
    }
}

int decode_max_pairs() { return kDecMaxPairs; }
int decode_max_tokens() { return kDecMaxTokens; }

template <int ACT, bool HAS_BIAS, int MAXC>
static void launch_gateup_t(const uint16_t* x, const uint16_t* w1, const float* b1, const int32_t* idx, uint16_t* glu,
                            int T, int H, int F, int E, int K, hipStream_t s) {
    dim3 grid(ceil_div(F, kDecFBlock), T * K);
    hipLaunchKernelGGL((moe_decode_gateup_kernel<ACT, HAS_BIAS, MAXC>), grid, dim3(kDecThreads), 0, s, x, w1, b1, idx,
                       glu, T, H, F, E, K);
}

template <bool HAS_BIAS, int MAXC>
static void launch_down_t(const uint16_t* glu, const uint16_t* w2, const float* b2, const int32_t* idx,
                          const float* route_w, uint16_t* out, int T, int H, int F, int E, int K, hipStream_t s) {
    dim3 grid(ceil_div(H, kDecRowsPerWaveD));
    hipLaunchKernelGGL((moe_decode_down_kernel<HAS_BIAS, MAXC>), grid, dim3(kDecThreads), 0, s, glu, w2, b2, idx,
                       route_w, out, T, H, F, E, K);
}

// MAXC = 16-byte chunks per lane per row = ceil(len / 512); supported up to 8 (len <= 4096).
static int pick_maxc(int len) {
    const int c = ceil_div(len, 8 * kWave);
    if (c <= 1) return 1;
    if (c <= 2) return 2;
    if (c <= 3) return 3;
    if (c <= 4) return 4;
    if (c <= 6) return 6;
    if (c <= 8) return 8;
    return -1;
}

#define CMOE_DEC_GU(ACT, BIAS, C) \
    case C: launch_gateup_t<ACT, BIAS, C>(x, w1, b1, idx, glu, T, H, F, E, K, s); break;
#define CMOE_DEC_GU_ALL(ACT, BIAS) \
    switch (cg) { CMOE_DEC_GU(ACT, BIAS, 1) CMOE_DEC_GU(ACT, BIAS, 2) CMOE_DEC_GU(ACT, BIAS, 3) \
                  CMOE_DEC_GU(ACT, BIAS, 4) CMOE_DEC_GU(ACT, BIAS, 6) CMOE_DEC_GU(ACT, BIAS, 8) default: break; }
#define CMOE_DEC_DN(BIAS, C) \
    case C: launch_down_t<BIAS, C>(glu, w2, b2, idx, route_w, out, T, H, F, E, K, s); break;
#define CMOE_DEC_DN_ALL(BIAS) \
    switch (cd) { CMOE_DEC_DN(BIAS, 1) CMOE_DEC_DN(BIAS, 2) CMOE_DEC_DN(BIAS, 3) CMOE_DEC_DN(BIAS, 4) \
                  CMOE_DEC_DN(BIAS, 6) CMOE_DEC_DN(BIAS, 8) default: break; }

bool decode_shape_supported(int H, int F) { return pick_maxc(H) > 0 && pick_maxc(F) > 0; }

hipError_t launch_decode(const uint16_t* x, const uint16_t* w1, const float* b1, const uint16_t* w2, const float* b2,
                         const int32_t* idx, const float* route_w, uint16_t* glu, uint16_t* out, int T, int H, int F,
                         int E, int K, int act, hipStream_t s, hipEvent_t* ev) {
    // ev (optional): 3 events recorded before gate_up, after gate_up, after down.
    auto mark = [&](int i) { if (ev) (void)hipEventRecord(ev[i], s); };
    const int cg = pick_maxc(H), cd = pick_maxc(F);
    mark(0);
    const bool bias = b1 != nullptr;
    if (act == kActSilu) {
        if (bias) { CMOE_DEC_GU_ALL(kActSilu, true) } else { CMOE_DEC_GU_ALL(kActSilu, false) }
    } else {
        if (bias) { CMOE_DEC_GU_ALL(kActGptOss, true) } else { CMOE_DEC_GU_ALL(kActGptOss, false) }
    }
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return st;
    mark(1);
    if (b2 != nullptr) { CMOE_DEC_DN_ALL(true) } else { CMOE_DEC_DN_ALL(false) }
    st = hipGetLastError();
    mark(2);
    return st;
}

}  // namespace cmoe
