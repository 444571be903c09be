// Token -> expert routing for the prefill path: histogram, exclusive-scan offsets, a stable
// permutation of the routed pairs grouped by expert, and the per-expert M-tile list that the
// grouped GEMMs schedule from.
//
// Replaces count_tokens_kernel (src/kops/cohere2_moe_experts/csrc/cohere2_moe_experts.cu:29-37),
// at::cumsum offsets (.cu:267-270) and build_perm_kernel (.cu:40-55). The reference's permutation
// is atomic-ordered and so varies run to run; this one is the op_eager order (expert, then top-k
// slot, then token), identical on every call.
//
// A classic radix-sort pass over the routed pairs visited in slot-major order q = k*T + t and cut
// into tiles of 1024:
//   count   (one workgroup per tile)  per-tile expert histogram -> counts[tile][E]
//   scan    (one workgroup)           per expert, exclusive scan over tiles (in place: the
//                                     absolute first write position of each tile), then over
//                                     experts -> offsets, tile list
//   (count and scan run as one single-workgroup launch while the per-tile histograms fit in LDS)
//   scatter (one workgroup per tile)  per-wave histograms inside the tile give each wave its
//                                     write cursors; each wave scatters its 256 pairs in order,
//                                     ranking lanes that share an expert with a bit-sliced ballot
// The scattered 4-byte writes of the permutation are spread over many CUs.
#include "moe_common.h"
#include "moe_split.h"

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

// Per-XCD item ranges of the packed GEMMs (moe_split.h), by all threads of the block: thread e
// holds expert e's pairs run at off and its nt M-tiles of BM rows at toff. Each thread writes the
// boundaries inside its expert (each of b[1..7] has exactly one writer when the list is not empty;
// for an empty one the clamp makes every bound 0 whatever s_b holds), then two threads clamp and
// store them.
__device__ __forceinline__ void write_xcd_split(const XcdSplit& sp, int BM, int run, int nt, int off, int toff,
                                                int valid_total, int tiles_total, int* s_b) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int g = 0; g < 2; ++g)
        split_expert(sp.fw[g], sp.n_tiles[g], BM, run, nt, toff, off,
                     32LL * sp.fw[g] * tiles_total + valid_total, s_b + 9 * g);
    __syncthreads();
    if (tid == 0 || tid == kWave) {
        const int g = tid == 0 ? 0 : 1;
        split_clamp(s_b + 9 * g, tiles_total * sp.n_tiles[g], sp.slots[g]);
        for (int k = 0; k < 9; ++k) sp.bounds[9 * g + k] = s_b[9 * g + k];
    }
}

constexpr int kRtTile = 1024;   // pairs per route tile
constexpr int kRtThreads = 256; // 4 waves x 256 pairs

// q / T for q = k*T + t with k < K <= 4096 (checked on the host): a float-reciprocal estimate is
// within 3*2^-24 * k < 1 of q / T, so the truncated estimate is off by at most one and a single
// exact integer correction fixes it. gfx950 has no integer divide; this replaces ~40 instructions.
__device__ __forceinline__ int div_by_t(int q, int T, float rT) {
    const int k = (int)((float)q * rT);
    const int r = q - k * T;
    return k + (r >= T ? 1 : 0) - (r < 0 ? 1 : 0);
}

__device__ __forceinline__ int expert_at(const int32_t* __restrict__ idx, int q, int T, int K, int E, float rT) {
    const int k = div_by_t(q, T, rT), t = q - k * T;
    const int v = idx[t * K + k];
    return ((unsigned)v < (unsigned)E) ? v : -1;
}

__global__ __launch_bounds__(kRtThreads) void moe_route_count_kernel(const int32_t* __restrict__ idx, int T, int K,
                                                                       int E, int32_t* __restrict__ counts) {
    extern __shared__ int32_t h[];  // [E]
    const int tid = threadIdx.x, P = T * K;
    const float rT = 1.0f / (float)T;
    for (int i = tid; i < E; i += kRtThreads) h[i] = 0;
    __syncthreads();
    const int q0 = blockIdx.x * kRtTile;
#pragma unroll 4
    for (int j = tid; j < kRtTile; j += kRtThreads) {
        const int q = q0 + j;
        if (q < P) {
            const int e = expert_at(idx, q, T, K, E, rT);
            if (e >= 0) atomicAdd(&h[e], 1);
        }
    }
    __syncthreads();
    for (int i = tid; i < E; i += kRtThreads) counts[(long long)blockIdx.x * E + i] = h[i];
}

// Work counters and completion flags of the grouped GEMMs that follow the route (zeroed here, so that
// no launch of its own is needed): kSchedInts ints, or none when sched is null.
constexpr int kSchedInts = 24;

__global__ __launch_bounds__(kRouteThreads) void moe_route_scan_kernel(int32_t* __restrict__ counts, int ntiles, int E,
                                                                        int BM, int32_t* __restrict__ offsets,
                                                                        int32_t* __restrict__ tile_offsets,
                                                                        int32_t* __restrict__ tile_expert,
                                                                        int32_t* __restrict__ meta,
                                                                        int32_t* __restrict__ sched, XcdSplit split) {
    __shared__ int wave_tot[kRouteWaves];
    __shared__ int s_split[18];
    const int tid = threadIdx.x;
    const int e = tid;  // E <= kRouteThreads is checked on the host
    int run = 0;
    if (e < E) {
#pragma unroll 8
        for (int t = 0; t < ntiles; ++t) {
            const int c = counts[(long long)t * E + e];
            counts[(long long)t * E + e] = run;
            run += c;
        }
    }
    int valid_total = 0, tiles_total = 0;
    const int off = block_exclusive_scan(run, wave_tot, &valid_total);
    const int nt = ceil_div(run, BM);
    const int toff = block_exclusive_scan(nt, wave_tot, &tiles_total);
    if (split.bounds) write_xcd_split(split, BM, run, nt, off, toff, valid_total, tiles_total, s_split);
    if (e < E) {
        offsets[e] = off;
        tile_offsets[e] = toff;
        for (int j = 0; j < nt; ++j) tile_expert[toff + j] = e;
#pragma unroll 8
        for (int t = 0; t < ntiles; ++t) counts[(long long)t * E + e] += off;  // absolute positions
    }
    if (tid == 0) {
        offsets[E] = valid_total;
        tile_offsets[E] = tiles_total;
        meta[0] = tiles_total;
        meta[1] = valid_total;
    }
    if (sched && tid < kSchedInts) sched[tid] = 0;
}

__global__ __launch_bounds__(kRtThreads) void moe_route_scatter_kernel(const int32_t* __restrict__ idx, int T, int K,
                                                                         int E, const int32_t* __restrict__ bases,
                                                                         int32_t* __restrict__ sorted_pairs,
                                                                         int8_t* __restrict__ row_zero) {
    extern __shared__ int32_t wh[];  // [4][E]: per-wave counts, then per-wave write cursors
    constexpr int kW = kRtThreads / kWave;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave, P = T * K;
    const float rT = 1.0f / (float)T;
    const int q0 = blockIdx.x * kRtTile + w * (kRtTile / kW);
    const int q1 = min(P, q0 + kRtTile / kW);
    for (int i = tid; i < kW * E; i += kRtThreads) wh[i] = 0;
    __syncthreads();
    int ex[kRtTile / kW / kWave];
#pragma unroll
    for (int c = 0; c < kRtTile / kW / kWave; ++c) {
        const int q = q0 + c * kWave + lane;
        ex[c] = q < q1 ? expert_at(idx, q, T, K, E, rT) : -1;
        if (ex[c] >= 0) atomicAdd(&wh[w * E + ex[c]], 1);
    }
    __syncthreads();
    const int32_t* tb = bases + (long long)blockIdx.x * E;
    for (int e = tid; e < E; e += kRtThreads) {
        int run = tb[e];
#pragma unroll
        for (int ww = 0; ww < kW; ++ww) {
            const int c = wh[ww * E + e];
            wh[ww * E + e] = run;
            run += c;
        }
    }
    __syncthreads();
    int nbits = 0;
    while ((1 << nbits) < E) ++nbits;
    const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
#pragma unroll
    for (int c = 0; c < kRtTile / kW / kWave; ++c) {
        const int q = q0 + c * kWave + lane;
        const int e = ex[c];
        const bool valid = e >= 0;
        uint64_t m = __ballot(valid);
        for (int b = 0; b < nbits; ++b) {
            const bool bit = valid && ((e >> b) & 1);
            const uint64_t bb = __ballot(bit);
            m &= bit ? bb : ~bb;
        }
        const int rank = __popcll(m & lt_mask);
        const int n_same = __popcll(m);
        const int base = valid ? wh[w * E + e] : 0;
        if (valid) {
            const int k = q / T, t = q - k * T;
            sorted_pairs[base + rank] = t * K + k;
            if (row_zero) row_zero[base + rank] = 0;
        }
        __builtin_amdgcn_wave_barrier();
        if (valid && rank == n_same - 1) wh[w * E + e] = base + n_same;
        __builtin_amdgcn_wave_barrier();
    }
}

// Count and scan fused in one workgroup: per-tile expert histograms are built in LDS with LDS
// atomics (thread t takes pairs t, t+1024, ... so iteration i is tile i), then scanned per expert
// over tiles and over experts exactly as in moe_route_scan_kernel. Used while the histograms fit in
// LDS (ntiles * E <= kRtFusedCells), which saves a launch and a pass over global memory.
constexpr int kRtFusedCells = 28 * 1024;

__global__ __launch_bounds__(kRouteThreads) void moe_route_count_scan_kernel(
    const int32_t* __restrict__ idx, int T, int K, int E, int BM, int ntiles, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ tile_offsets, int32_t* __restrict__ tile_expert,
    int32_t* __restrict__ meta, int32_t* __restrict__ sched, XcdSplit split) {
    __shared__ int32_t h[kRtFusedCells];  // [ntiles][E]
    __shared__ int wave_tot[kRouteWaves];
    __shared__ int s_split[18];
    const int tid = threadIdx.x, P = T * K;  // P <= kRtFusedCells * kRtTile here, far below 2^31
    for (int i = tid; i < ntiles * E; i += kRouteThreads) h[i] = 0;
    __syncthreads();
    // idx is read in memory order (pair i = t*K + k), four consecutive pairs per thread and chunk, so
    // a wave's load touches 8 cache lines rather than one per lane; each pair is then counted in the
    // tile of its slot-major position q = k*T + t. (t, k) of a chunk's first pair come from one
    // exact division (double reciprocal: quotient < 2^31, error < 1, one correction), then k steps.
    const double rK = 1.0 / (double)K;
    const int nchunks = ceil_div(P, 4);
    for (int c0 = tid; c0 < nchunks; c0 += 8 * kRouteThreads) {
        int ev[8][4];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = 4 * (c0 + u * kRouteThreads);
#pragma unroll
            for (int v = 0; v < 4; ++v) ev[u][v] = i + v < P ? idx[i + v] : -1;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = 4 * (c0 + u * kRouteThreads);
            if (i >= P) continue;
            int t = (int)((double)i * rK), k = i - t * K;
            t += (k >= K ? 1 : 0) - (k < 0 ? 1 : 0);
            k = i - t * K;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int e = ev[u][v];
                if ((unsigned)e < (unsigned)E) atomicAdd(&h[((k * T + t) / kRtTile) * E + e], 1);
                if (++k == K) {
                    k = 0;
                    ++t;
                }
            }
        }
    }
    __syncthreads();
    const int e = tid;  // E <= kRouteThreads is checked on the host
    int run = 0;
    if (e < E) {
        for (int t = 0; t < ntiles; ++t) {
            const int c = h[t * E + e];
            h[t * E + e] = run;
            run += c;
        }
    }
    int valid_total = 0, tiles_total = 0;
    const int off = block_exclusive_scan(run, wave_tot, &valid_total);
    const int nt = ceil_div(run, BM);
    const int toff = block_exclusive_scan(nt, wave_tot, &tiles_total);
    if (split.bounds) write_xcd_split(split, BM, run, nt, off, toff, valid_total, tiles_total, s_split);
    if (e < E) {
        offsets[e] = off;
        tile_offsets[e] = toff;
        for (int j = 0; j < nt; ++j) tile_expert[toff + j] = e;
        for (int t = 0; t < ntiles; ++t) counts[t * E + e] = h[t * E + e] + off;  // absolute positions
    }
    if (tid == 0) {
        offsets[E] = valid_total;
        tile_offsets[E] = tiles_total;
        meta[0] = tiles_total;
        meta[1] = valid_total;
    }
    if (sched && tid < kSchedInts) sched[tid] = 0;
}

// The whole route in one launch: workgroup b < ntiles (1024 threads) owns route tile b. Every workgroup
// builds all tiles' expert histograms in LDS and scans them (the same work as
// moe_route_count_scan_kernel, repeated per workgroup: idx is small and L2-resident), which gives it
// the absolute first write position of each expert in its own tile. Then each of its 16 waves takes 64
// consecutive pairs of the tile: per-wave histograms give the write cursors, and lanes that share an
// expert are ranked with a bit-sliced ballot, exactly as in the scatter kernel. One more workgroup
// (b = ntiles) writes the offsets, the tile list, the GEMMs' XCD split and counters from the same scans
// and scatters nothing, so those writes run beside the scatter instead of after it in one workgroup
// (measured: the workgroup that did both ended the launch ~2.5 us after the others). Output identical
// to the two-launch route.
constexpr int kRtChunks = 8;           // 16-byte idx chunks per thread and round of the histogram pass
constexpr int kRtOneCells = 39 * 1024;  // LDS cells: ntiles * E histograms + 16 * E wave cursors (156 KiB)

__global__ __launch_bounds__(kRouteThreads) void moe_route_one_kernel(
    const int32_t* __restrict__ idx, int T, int K, int E, int BM, int ntiles, int32_t* __restrict__ offsets,
    int32_t* __restrict__ sorted_pairs, int32_t* __restrict__ tile_offsets, int32_t* __restrict__ tile_expert,
    int32_t* __restrict__ meta, int32_t* __restrict__ sched, int8_t* __restrict__ row_zero, XcdSplit split) {
    extern __shared__ int32_t rt_lds[];
    __shared__ int s_split[18];
    int32_t* h = rt_lds;                    // [ntiles][E]
    int32_t* wc = rt_lds + ntiles * E;      // [16][E] per-wave counts, then cursors
    __shared__ int wave_tot[kRouteWaves];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), P = T * K;
    const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
    const bool writer = blockIdx.x == (unsigned)ntiles;  // offsets, tile list, split; owns no tile
    const float rT = 1.0f / (float)T;
    for (int i = tid; i < (ntiles + kRouteWaves) * E; i += kRouteThreads) rt_lds[i] = 0;
    const int q = blockIdx.x * kRtTile + w * kWave + lane;
    const int eq = q < P ? expert_at(idx, q, T, K, E, rT) : -1;
    __syncthreads();
    const double rK = 1.0 / (double)K;
    const int nchunks = ceil_div(P, 4);
    // idx in 16-byte chunks through a buffer descriptor (P * 4 < 2^31 on this path): one load
    // instruction per chunk, the tail of the last chunk reads 0 and is masked by i + v < P
    const __amdgpu_buffer_rsrc_t ridx = __builtin_amdgcn_make_buffer_rsrc((void*)idx, (short)0, P * 4, kBufferWord3);
    for (int c0 = tid; c0 < nchunks; c0 += kRtChunks * kRouteThreads) {
        u32x4 ev[kRtChunks];
#pragma unroll
        for (int u = 0; u < kRtChunks; ++u)
            ev[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  ridx, (uint32_t)(c0 + u * kRouteThreads) * 16u, 0, 0));
#pragma unroll
        for (int u = 0; u < kRtChunks; ++u) {
            const int i = 4 * (c0 + u * kRouteThreads);
            if (i >= P) continue;
            int t = (int)((double)i * rK), k = i - t * K;
            t += (k >= K ? 1 : 0) - (k < 0 ? 1 : 0);
            k = i - t * K;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int e = (int)ev[u][v];
                if (i + v < P && (unsigned)e < (unsigned)E) atomicAdd(&h[((k * T + t) / kRtTile) * E + e], 1);
                if (++k == K) {
                    k = 0;
                    ++t;
                }
            }
        }
    }
    if (eq >= 0) atomicAdd(&wc[w * E + eq], 1);
    __syncthreads();
    const int e = tid;  // E <= kRouteThreads is checked on the host
    int run = 0, mine = 0;
    if (e < E) {
        for (int t = 0; t < ntiles; ++t) {
            const int c = h[t * E + e];
            if (t == (int)blockIdx.x) mine = run;
            run += c;
        }
    }
    int valid_total = 0, tiles_total = 0;
    const int off = block_exclusive_scan(run, wave_tot, &valid_total);
    const int nt = ceil_div(run, BM);
    const int toff = block_exclusive_scan(nt, wave_tot, &tiles_total);
    if (writer) {  // uniform over the workgroup (write_xcd_split synchronises it)
        if (split.bounds) write_xcd_split(split, BM, run, nt, off, toff, valid_total, tiles_total, s_split);
        if (e < E) {
            offsets[e] = off;
            tile_offsets[e] = toff;
            for (int j = 0; j < nt; ++j) tile_expert[toff + j] = e;
        }
        if (tid == 0) {
            offsets[E] = valid_total;
            tile_offsets[E] = tiles_total;
            meta[0] = tiles_total;
            meta[1] = valid_total;
        }
        if (sched && tid < kSchedInts) sched[tid] = 0;
        return;
    }
    if (e < E) {
        int cur = off + mine;
#pragma unroll
        for (int ww = 0; ww < kRouteWaves; ++ww) {
            const int c = wc[ww * E + e];
            wc[ww * E + e] = cur;
            cur += c;
        }
    }
    __syncthreads();
    int nbits = 0;
    while ((1 << nbits) < E) ++nbits;
    const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
    const bool valid = eq >= 0;
    uint64_t m = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
        const bool bit = valid && ((eq >> b) & 1);
        const uint64_t bb = __ballot(bit);
        m &= bit ? bb : ~bb;
    }
    if (valid) {
        const int k = div_by_t(q, T, rT), t = q - k * T;
        const int pos = wc[w * E + eq] + __popcll(m & lt_mask);
        sorted_pairs[pos] = t * K + k;
        if (row_zero) row_zero[pos] = 0;
    }
}

int route_tiles(int T, int K) { return ceil_div(T * K, kRtTile); }
size_t route_workspace_bytes(int T, int K, int E) { return (size_t)max(route_tiles(T, K), 1) * E * sizeof(int32_t); }

hipError_t launch_route(const int32_t* idx, int T, int K, int E, int BM, int32_t* offsets, int32_t* sorted_pairs,
                        int32_t* tile_offsets, int32_t* tile_expert, int32_t* meta, int32_t* counts,
                        int32_t* sched, hipStream_t stream, int8_t* row_zero, const XcdSplit* split) {
    const int nt = route_tiles(T, K);
    const XcdSplit sp = split ? *split : XcdSplit{};
    if (nt > 0 && (long long)(nt + kRouteWaves) * E <= kRtOneCells) {
        static bool lds_attr = false;  // dynamic LDS above 64 KiB must be allowed once per process
        if (!lds_attr) {
            const hipError_t st = hipFuncSetAttribute((const void*)moe_route_one_kernel,
                                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                                      kRtOneCells * (int)sizeof(int32_t));
            if (st != hipSuccess) return st;
            lds_attr = true;
        }
        hipLaunchKernelGGL(moe_route_one_kernel, dim3(nt + 1), dim3(kRouteThreads),
                           (size_t)(nt + kRouteWaves) * E * sizeof(int32_t), stream, idx, T, K, E, BM, nt, offsets,
                           sorted_pairs, tile_offsets, tile_expert, meta, sched, row_zero, sp);
        return hipGetLastError();
    }
    if ((long long)nt * E <= kRtFusedCells) {
        hipLaunchKernelGGL(moe_route_count_scan_kernel, dim3(1), dim3(kRouteThreads), 0, stream, idx, T, K, E, BM, nt,
                           counts, offsets, tile_offsets, tile_expert, meta, sched, sp);
    } else {
        hipLaunchKernelGGL(moe_route_count_kernel, dim3(nt), dim3(kRtThreads), E * sizeof(int32_t), stream, idx, T, K,
                           E, counts);
        hipLaunchKernelGGL(moe_route_scan_kernel, dim3(1), dim3(kRouteThreads), 0, stream, counts, nt, E, BM, offsets,
                           tile_offsets, tile_expert, meta, sched, sp);
    }
    if (nt > 0)
        hipLaunchKernelGGL(moe_route_scatter_kernel, dim3(nt), dim3(kRtThreads), 4 * E * sizeof(int32_t), stream, idx,
                           T, K, E, counts, sorted_pairs, row_zero);
    return hipGetLastError();
}

}  // namespace cmoe
