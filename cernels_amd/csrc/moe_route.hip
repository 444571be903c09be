// Token -> expert routing for the prefill path: histogram, exclusive-scan offsets, a stable
// permutation of the routed pairs grouped by expert, and the per-expert M-tile list that the
// grouped GEMMs schedule from.
//
// Replaces, in one launch and without atomics on the output order:
//   count_tokens_kernel (src/kops/cohere2_moe_experts/csrc/cohere2_moe_experts.cu:29-37),
//   at::cumsum offsets (.cu:267-270) and build_perm_kernel (.cu:40-55).
// The reference's permutation is atomic-ordered and so varies run to run; this one is the
// op_eager order (expert, then top-k slot, then token), identical on every call.
//
// One workgroup of 1024 threads (16 waves). The routed pairs are visited in slot-major order
// q = k*T + t, cut into 16 contiguous segments, one per wave. Each wave histograms its segment
// into LDS; per-(wave, expert) bases come from a scan over waves then experts; each wave then
// scatters its segment in order, ranking lanes that share an expert with a bit-sliced ballot.
#include "moe_common.h"

namespace cmoe {

constexpr int kRouteThreads = 1024;
constexpr int kRouteWaves = kRouteThreads / kWave;

// Exclusive scan of one int per thread over the 1024-thread block; *total gets the sum.
__device__ __forceinline__ int block_exclusive_scan(int v, int* wave_tot, int* total) {
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    int x = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        int y = __shfl_up(x, o, kWave);
        if (lane >= o) x += y;
    }
    if (lane == kWave - 1) wave_tot[w] = x;
    __syncthreads();
    if (w == 0) {
        int s = lane < kRouteWaves ? wave_tot[lane] : 0;
#pragma unroll
        for (int o = 1; o < kRouteWaves; o <<= 1) {
            int y = __shfl_up(s, o, kWave);
            if (lane >= o) s += y;
        }
        if (lane < kRouteWaves) wave_tot[lane] = s;  // inclusive wave prefix
    }
    __syncthreads();
    const int before = w > 0 ? wave_tot[w - 1] : 0;
    *total = wave_tot[kRouteWaves - 1];
    __syncthreads();  // wave_tot is reused by the next scan
    return before + x - v;
}

constexpr uint16_t kNoExpert = 0xffff;

// STAGED: every expert id is first copied into LDS as uint16 in slot-major order (coalesced,
// many loads in flight); the histogram and scatter phases then never touch global memory.
template <bool STAGED>
__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(
    const int32_t* __restrict__ idx, int T, int K, int E, int BM, int32_t* __restrict__ offsets,
    int32_t* __restrict__ sorted_pairs, int32_t* __restrict__ tile_offsets, int32_t* __restrict__ tile_expert,
    int32_t* __restrict__ meta) {
    extern __shared__ int32_t hist[];  // [kRouteWaves][E], then (STAGED) uint16 ids [P]
    __shared__ int wave_tot[kRouteWaves];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
    const int P = T * K;
    uint16_t* eid = reinterpret_cast<uint16_t*>(hist + kRouteWaves * E);

    for (int i = tid; i < kRouteWaves * E; i += kRouteThreads) hist[i] = 0;
    if constexpr (STAGED) {
#pragma unroll 8
        for (int i = tid; i < P; i += kRouteThreads) {
            const int v = idx[i];
            const int t = i / K, k = i - t * K;
            eid[k * T + t] = ((unsigned)v < (unsigned)E) ? (uint16_t)v : kNoExpert;
        }
    }
    __syncthreads();
    // expert id of slot-major pair q (-1 if out of range)
    auto expert_at = [&](int q) -> int {
        if constexpr (STAGED) {
            const uint16_t v = eid[q];
            return v == kNoExpert ? -1 : (int)v;
        } else {
            const int k = q / T, t = q - k * T;
            const int v = idx[t * K + k];
            return ((unsigned)v < (unsigned)E) ? v : -1;
        }
    };

    const int seg = ceil_div(ceil_div(P, kRouteWaves), kWave) * kWave;
    const int q0 = min(P, w * seg), q1 = min(P, q0 + seg);

    // 1. per-wave histogram (order-free, so LDS atomics are fine here)
    for (int q = q0 + lane; q < q1; q += kWave) {
        const int e = expert_at(q);
        if (e >= 0) atomicAdd(&hist[w * E + e], 1);
    }
    __syncthreads();

    // 2. bases: over waves within an expert, then over experts; tile counts alike
    const int e = tid;  // E <= kRouteThreads is checked on the host
    int cnt = 0;
    if (e < E) {
        for (int ww = 0; ww < kRouteWaves; ++ww) {
            const int c = hist[ww * E + e];
            hist[ww * E + e] = cnt;
            cnt += c;
        }
    }
    int valid_total = 0, tiles_total = 0;
    const int off = block_exclusive_scan(cnt, wave_tot, &valid_total);
    const int ntiles = ceil_div(cnt, BM);
    const int toff = block_exclusive_scan(ntiles, wave_tot, &tiles_total);
    if (e < E) {
        offsets[e] = off;
        tile_offsets[e] = toff;
        for (int ww = 0; ww < kRouteWaves; ++ww) hist[ww * E + e] += off;  // absolute write cursors
        for (int j = 0; j < ntiles; ++j) tile_expert[toff + j] = e;
    }
    if (tid == 0) {
        offsets[E] = valid_total;
        tile_offsets[E] = tiles_total;
        meta[0] = tiles_total;
        meta[1] = valid_total;
    }
    __syncthreads();

    // 3. stable scatter, one wave per segment, 64 pairs at a time in order
    int nbits = 0;
    while ((1 << nbits) < E) ++nbits;
    const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
    for (int qb = q0; qb < q1; qb += kWave) {
        const int q = qb + lane;
        int ex = -1, p = 0;
        if (q < q1) {
            const int k = q / T, t = q - k * T;
            p = t * K + k;
            ex = expert_at(q);
        }
        const bool valid = ex >= 0;
        uint64_t m = __ballot(valid);
        for (int b = 0; b < nbits; ++b) {
            const bool bit = valid && ((ex >> b) & 1);
            const uint64_t bb = __ballot(bit);
            m &= bit ? bb : ~bb;
        }
        const int rank = __popcll(m & lt_mask);
        const int n_same = __popcll(m);
        const int base = valid ? hist[w * E + ex] : 0;
        if (valid) sorted_pairs[base + rank] = p;
        __builtin_amdgcn_wave_barrier();
        if (valid && rank == n_same - 1) hist[w * E + ex] = base + n_same;
        __builtin_amdgcn_wave_barrier();
    }
}

static size_t route_hist_bytes(int E) { return (size_t)kRouteWaves * E * sizeof(int32_t); }

static int max_lds_per_block() {
    static int v = 0;
    if (v == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && n > 0)
            v = n;
        else
            v = 64 * 1024;
    }
    return v;
}

hipError_t launch_route(const int32_t* idx, int T, int K, int E, int BM, int32_t* offsets, int32_t* sorted_pairs,
                        int32_t* tile_offsets, int32_t* tile_expert, int32_t* meta, hipStream_t stream) {
    const int cap = max_lds_per_block() - 1024;  // room for the static wave totals
    const size_t staged = route_hist_bytes(E) + (((size_t)T * K * sizeof(uint16_t) + 3) & ~(size_t)3);
    static bool attr_staged = false, attr_plain = false;
    if (staged <= (size_t)cap) {
        if (!attr_staged) {
            hipError_t st = hipFuncSetAttribute((const void*)moe_route_kernel<true>,
                                                hipFuncAttributeMaxDynamicSharedMemorySize, cap);
            if (st != hipSuccess) return st;
            attr_staged = true;
        }
        hipLaunchKernelGGL(moe_route_kernel<true>, dim3(1), dim3(kRouteThreads), staged, stream, idx, T, K, E, BM,
                           offsets, sorted_pairs, tile_offsets, tile_expert, meta);
    } else {
        if (!attr_plain) {
            hipError_t st = hipFuncSetAttribute((const void*)moe_route_kernel<false>,
                                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                                (int)route_hist_bytes(kRouteThreads));
            if (st != hipSuccess) return st;
            attr_plain = true;
        }
        hipLaunchKernelGGL(moe_route_kernel<false>, dim3(1), dim3(kRouteThreads), route_hist_bytes(E), stream, idx, T,
                           K, E, BM, offsets, sorted_pairs, tile_offsets, tile_expert, meta);
    }
    return hipGetLastError();
}

}  // namespace cmoe
