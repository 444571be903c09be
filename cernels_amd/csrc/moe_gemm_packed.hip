// Prefill grouped GEMMs over expert weights packed in MFMA-fragment order (bf16 MFMA, gfx950).
//
// Same mathematics as the grouped GEMMs on the transformers layouts (moe_gemm.hip):
//   GEMM1  glu[r, :] = act( X[tok(r), :] · W1_e + b1_e )        SwiGLU / gpt-oss gate in the epilogue
//   GEMM2  Y[p, :]   = w_p · ( glu[r, :] · W2_e + b2_e )        routing weight in the epilogue (fp32)
// and the same route kernel, item list and deterministic k-sum combine. What changes is how the
// weights reach the matrix cores. The weights are re-laid once (cernels_moe_pack_weights) so that
// each 32x16 MFMA operand fragment is 1 KB of contiguous memory in exactly the order a wave's lanes
// consume it. A wave then streams its weight columns straight into registers with one contiguous
// 1 KB read per fragment: every HBM request is a full, sequential line run, nothing of the weights
// goes through LDS, and how many bytes are in flight is bounded by registers rather than by LDS.
// Only the activation tile (token rows gathered through the expert-sorted pair list) is staged in
// LDS, since all four waves of a workgroup share it.
//
// Workgroup: 8 waves, two per SIMD, one workgroup per CU. Each wave owns one 64-column group of the
// N-tile (GEMM1: 32 gate + the 32 matching up columns; GEMM2: 64 output columns) for all 128 rows of
// the item, so every weight fragment is loaded once per workgroup and used by 4 MFMAs. All waves
// skip the item's empty 32-row blocks, so an item of fewer than 128 rows costs MFMA time in
// proportion to its rows. K advances in stages of 64: weight loads are issued one stage,
// activation loads two stages before their MFMAs.
#include <type_traits>

#include "moe_tile.h"

namespace cmoe {

constexpr int kPkWaves = 8;                 // waves per workgroup = column groups per N-tile
constexpr int kPkThreads = kPkWaves * kWave;
constexpr int kPkBM = 128;
constexpr int kPkMB = kPkBM / 32;           // 32-row MFMA blocks per item
constexpr int kPkABytes = kPkBM * kBK * 2;  // 16 KB A stage
constexpr int kPkFrag = 512;                // bf16 elements of one fragment (1 KB)
constexpr int kPkEpiStride = kPkWaves * 32 + 8;  // bf16 row stride of the GEMM1 output tile in LDS

constexpr int kModePkGateUp = 0;
constexpr int kModePkDown = 1;

// Packed layout of one projection, viewed as B[k][n] (reduction length Kd, KS = Kd/16 k-steps) with
// NG column groups of two 32-column fragments:
//   gate_up: group g = glu columns [32g, 32g+32); fragment 0 = gate, 1 = up.  Kd = H, NG = F/32.
//   down:    group g = output columns [64g, 64g+64); fragment f = [64g+32f, +32). Kd = F, NG = H/64.
// Groups are bundled by four (an N-tile: one group per wave) and stored k-step-major inside a tile, so
// the four waves of a workgroup read one contiguous 8 KB run per k-step. Lane l of fragment
// (g, ks, f) holds B[16ks + 8(l/32) + j][column l%32 of the fragment], j = 0..7.
// Returns the fragment's index in 1 KB units.
__host__ __device__ inline long long packed_frag(int e, int g, int ks, int f, int NG, int KS) {
    const int t = g >> 2, w = g & 3, nw = min(4, NG - 4 * t);
    return ((long long)e * NG * KS + 4LL * KS * t + (long long)ks * nw + w) * 2 + f;
}

// ---- packing (one-time, per weight tensor) ---------------------------------------------------------
// One thread per 16-byte lane chunk of the packed output, in logical (e, g, ks, f, lane) order.
template <int WHICH, int LAYOUT>
__global__ __launch_bounds__(256) void moe_pack_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                       int E, int H, int F) {
    const int Kd = WHICH == 0 ? H : F;
    const int NG = WHICH == 0 ? F / 32 : H / 64;
    const int KS = Kd / 16;
    const long long total = (long long)E * NG * KS * 2 * kWave;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int lane = (int)(i % kWave);
    long long q = i / kWave;
    const int f = (int)(q % 2);
    q /= 2;
    const int ks = (int)(q % KS);
    q /= KS;
    const int g = (int)(q % NG);
    const int e = (int)(q / NG);
    const int k0 = 16 * ks + 8 * (lane >> 5);
    const int c = lane & 31;
    u32x4 v;
    if constexpr (WHICH == 0) {
        const int fc = 32 * g + c;  // intermediate index
        if constexpr (LAYOUT == kLayoutConcat) {  // [E, 2F, H]: gate row fc, up row F + fc
            v = *reinterpret_cast<const u32x4*>(src + ((long long)e * 2 * F + f * F + fc) * H + k0);
        } else {  // [E, H, 2F]: gate column 2fc, up column 2fc + 1
            uint16_t t[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) t[j] = src[((long long)e * H + k0 + j) * 2 * F + 2 * fc + f];
            v = u32x4{t[0] | (uint32_t)t[1] << 16, t[2] | (uint32_t)t[3] << 16, t[4] | (uint32_t)t[5] << 16,
                      t[6] | (uint32_t)t[7] << 16};
        }
    } else {
        const int n = 64 * g + 32 * f + c;  // output (hidden) index
        if constexpr (LAYOUT == kLayoutConcat) {  // [E, H, F]
            v = *reinterpret_cast<const u32x4*>(src + ((long long)e * H + n) * F + k0);
        } else {  // [E, F, H]
            uint16_t t[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) t[j] = src[((long long)e * F + k0 + j) * H + n];
            v = u32x4{t[0] | (uint32_t)t[1] << 16, t[2] | (uint32_t)t[3] << 16, t[4] | (uint32_t)t[5] << 16,
                      t[6] | (uint32_t)t[7] << 16};
        }
    }
    *reinterpret_cast<u32x4*>(dst + packed_frag(e, g, ks, f, NG, KS) * kPkFrag + lane * 8) = v;
}

size_t packed_weight_bytes(int H, int F, int E, int which) {
    (void)which;  // both projections keep their element count: 2FH (gate_up) and HF (down)
    return which == 0 ? (size_t)E * 2 * F * H * 2 : (size_t)E * H * F * 2;
}

hipError_t launch_pack(const uint16_t* src, uint16_t* dst, int E, int H, int F, int layout, int which, hipStream_t s) {
    const long long chunks = (long long)E * (which == 0 ? 2LL * F * H : (long long)H * F) / 8;
    const unsigned grid = (unsigned)((chunks + 255) / 256);
    if (which == 0) {
        if (layout == kLayoutConcat) hipLaunchKernelGGL((moe_pack_kernel<0, kLayoutConcat>), dim3(grid), dim3(256), 0, s, src, dst, E, H, F);
        else hipLaunchKernelGGL((moe_pack_kernel<0, kLayoutInterleaved>), dim3(grid), dim3(256), 0, s, src, dst, E, H, F);
    } else {
        if (layout == kLayoutConcat) hipLaunchKernelGGL((moe_pack_kernel<1, kLayoutConcat>), dim3(grid), dim3(256), 0, s, src, dst, E, H, F);
        else hipLaunchKernelGGL((moe_pack_kernel<1, kLayoutInterleaved>), dim3(grid), dim3(256), 0, s, src, dst, E, H, F);
    }
    return hipGetLastError();
}

// ---- the grouped GEMM ------------------------------------------------------------------------------

struct PkParams {
    const uint16_t* A;             // GEMM1: x [T, H]; GEMM2: glu [P, F] (rows in expert order)
    const uint16_t* B;             // packed weights of this projection
    const float* bias;             // GEMM1: [E, 2F]; GEMM2: [E, H]; or null
    const int32_t* sorted_pairs;   // [P]
    const int32_t* offsets;        // [E+1]
    const int32_t* tile_offsets;   // [E+1]
    const int32_t* tile_expert;    // [tiles]
    const int32_t* meta;           // [0] = M-tiles
    const float* route_w;          // [P] (GEMM2)
    void* out;                     // GEMM1: glu bf16 [P, F]; GEMM2: Y fp32 [P, H]
    int Kd, NG, KS, n_tiles;
    int F, H, topk;
    int bias_interleaved;          // GEMM1 bias order: 0 = [gate F | up F], 1 = gate/up interleaved
};

template <int N>
using IC = std::integral_constant<int, N>;


template <int MODE, int ACT, bool HAS_BIAS>
__global__ __launch_bounds__(kPkThreads, 1) void moe_gemm_packed_kernel(PkParams prm) {
    __shared__ __attribute__((aligned(16))) unsigned char smem[2 * kPkABytes];
    __shared__ int s_pair[kPkBM];
    __shared__ float s_w[kPkBM];
    __shared__ __attribute__((aligned(16))) uint16_t s_epi[MODE == kModePkGateUp ? kPkBM * kPkEpiStride : 8];
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);

    const int tiles = prm.meta[0];
    const int total = tiles * prm.n_tiles;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, slots = gridDim.x >> 3;
    const int per = ceil_div(total, 8);
    const int it_end = min(total, (xcd + 1) * per);
    const int Kd = prm.Kd, nst = Kd / kBK;

    // Items of XCD x are [x*per, x*per + per), handed to its slots in snake order (slot s takes
    // s, 2*slots-1-s, 2*slots+s, ...) so that long and short items mix on every CU, while the items
    // that share a weight tile (neighbours in the list) still run at the same time on one XCD.
    for (int j = 0;; ++j) {
        const int off = (j & 1) ? (j + 1) * slots - 1 - slot : j * slots + slot;
        const int it = xcd * per + off;
        if (off >= per || it >= it_end) break;
        const WorkItem wi = decode_item(it, prm.n_tiles, kPkBM, prm.tile_expert, prm.tile_offsets, prm.offsets);
        const int e = wi.e, row_begin = wi.row_begin, rows = wi.rows;
        const int g = wi.n_idx * kPkWaves + wave;
        const int nmb = ceil_div(rows, 32);  // non-empty 32-row blocks
        const bool active = g < prm.NG;      // wave-uniform: this wave stores results

        __syncthreads();  // the previous item is done with the LDS buffers and the pair table
        if constexpr (MODE == kModePkDown) {
            if (tid < rows) {
                const int p = prm.sorted_pairs[row_begin + tid];
                s_pair[tid] = p;
                s_w[tid] = prm.route_w[p];
            }
        }
        // A rows: thread t loads 16-byte chunk t%8 of rows t/8 and t/8 + 64 of each stage; a wave
        // instruction covers 8 rows x 128 B.
        const int a_chunk = tid & 7;
        const uint16_t* a_src[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int ra = min((tid >> 3) + 64 * i, rows - 1);
            long long src_row;
            if constexpr (MODE == kModePkGateUp) src_row = prm.sorted_pairs[row_begin + ra] / prm.topk;
            else src_row = row_begin + ra;
            a_src[i] = prm.A + src_row * Kd + a_chunk * 8;
        }
        const int gc = g < prm.NG ? g : wi.n_idx * kPkWaves;  // idle waves read the tile's first group
        const int nw = min(4, prm.NG - 4 * (gc >> 2));
        const uint16_t* b_ptr = prm.B + packed_frag(e, gc, 0, 0, prm.NG, prm.KS) * kPkFrag + lane * 8;
        const long long b_step = (long long)nw * 2 * kPkFrag;  // elements between consecutive k-steps

        f32x16 acc[kPkMB][2];
#pragma unroll
        for (int mb = 0; mb < kPkMB; ++mb)
#pragma unroll
            for (int f = 0; f < 2; ++f)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[mb][f][r] = 0.f;

        // Activation chunks in a two-slot register ring (loaded two stages before their MFMAs,
        // written to LDS one stage before); weight fragments in one slot per k-step, refilled with the
        // next stage's k-step as soon as its MFMAs have read it (one stage ahead). Every load is visible to the compiler, which waits for exactly the loads each
        // use needs. Loads are never behind a branch, so those waits stay exact: past the last stage
        // a step re-reads the last stage (an L2 hit), and a wave whose column group is past the end
        // loads valid fragments of the tile, skips its MFMAs and stores nothing.
        u32x4 aring[2][2];
        u32x4 breg[4][2];  // k-step q of the current stage, refilled with k-step q of the next
        auto load_a = [&](int s, auto rc) {
            constexpr int r = decltype(rc)::value;
            const int sc = min(s, nst - 1);
#pragma unroll
            for (int i = 0; i < 2; ++i) aring[r][i] = *reinterpret_cast<const u32x4*>(a_src[i] + sc * kBK);
        };
        auto load_b = [&](int s, int q) {  // k-step q of stage s
            const uint16_t* bp = b_ptr + (long long)(4 * min(s, nst - 1) + q) * b_step;
#pragma unroll
            for (int f = 0; f < 2; ++f) breg[q][f] = *reinterpret_cast<const u32x4*>(bp + f * kPkFrag);
        };
        auto store_a = [&](auto rc) {  // activation chunks of ring slot r -> LDS buffer r
            constexpr int r = decltype(rc)::value;
            unsigned char* sA = smem + r * kPkABytes;
#pragma unroll
            for (int i = 0; i < 2; ++i)
                *reinterpret_cast<u32x4*>(sA + lds_off((tid >> 3) + 64 * i, a_chunk)) = aring[r][i];
        };
        auto kloop = [&](auto nmbc) {
            constexpr int NMB = decltype(nmbc)::value;
            // One A fragment register per 32-row block: right after the two MFMAs of block mb at
            // k-step q consume it, it is reloaded with block mb's fragment of k-step q + 1, which then
            // has the other blocks' MFMAs to arrive. The next stage's weight loads are spread over the
            // four k-steps (fenced with sched_barrier) so that the CU's address unit works on them
            // while the matrix cores run, instead of all waves queueing their loads at once.
            auto step = [&](int s, auto c0, auto c1) {
                constexpr int b = decltype(c0)::value;
                __syncthreads();  // stage s is in LDS buffer b; every wave is done with the other buffer
                const unsigned char* sA = smem + b * kPkABytes;
                auto read_af = [&](int q, int mb) {
                    return *reinterpret_cast<const bf16x8*>(sA + lds_off(mb * 32 + (lane & 31), 2 * q + (lane >> 5)));
                };
                load_a(s + 2, c0);  // into the slot stage s's chunks left
                bf16x8 af[NMB];
#pragma unroll
                for (int mb = 0; mb < NMB; ++mb) af[mb] = read_af(0, mb);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    __builtin_amdgcn_sched_barrier(0);
                    const bf16x8 b0 = __builtin_bit_cast(bf16x8, breg[q][0]);
                    const bf16x8 b1 = __builtin_bit_cast(bf16x8, breg[q][1]);
#pragma unroll
                    for (int mb = 0; mb < NMB; ++mb) {
                        if (active) {  // wave-uniform, no loads inside: the compiler's waits stay exact
                            acc[mb][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mb], b0, acc[mb][0], 0, 0, 0);
                            acc[mb][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mb], b1, acc[mb][1], 0, 0, 0);
                        }
                        if (q + 1 < 4) af[mb] = read_af(q + 1, mb);
                    }
                    load_b(s + 1, q);  // k-step q of the next stage into the registers just consumed
                }
                __builtin_amdgcn_sched_barrier(0);
                store_a(c1);  // stage s+1's chunks -> the other LDS buffer
            };
            load_a(0, IC<0>{});
            load_a(1, IC<1>{});
#pragma unroll
            for (int q = 0; q < 4; ++q) load_b(0, q);
            store_a(IC<0>{});
            int s = 0;
            for (; s + 1 < nst; s += 2) {
                step(s, IC<0>{}, IC<1>{});
                step(s + 1, IC<1>{}, IC<0>{});
            }
            if (s < nst) step(s, IC<0>{}, IC<1>{});
        };
        switch (nmb) {
            case 1: kloop(IC<1>{}); break;
            case 2: kloop(IC<2>{}); break;
            case 3: kloop(IC<3>{}); break;
            default: kloop(IC<4>{}); break;
        }

        // ---- epilogue. Element r of a 32x32 accumulator block is at row 8*(r/4) + 4*(lane/32) + (r%4),
        // column lane & 31.
        if constexpr (MODE == kModePkGateUp) {
            // SwiGLU in registers, the bf16 tile staged in LDS, then written as 16-byte chunks: each
            // output row of the N-tile is one contiguous 512-byte run.
            if (active) {
                const int fcol = 32 * g + (lane & 31);
                float bg = 0.f, bu = 0.f;
                if constexpr (HAS_BIAS) {
                    const float* be = prm.bias + (long long)e * 2 * prm.F;
                    bg = prm.bias_interleaved ? be[2 * fcol] : be[fcol];
                    bu = prm.bias_interleaved ? be[2 * fcol + 1] : be[prm.F + fcol];
                }
                uint16_t* ep = s_epi + wave * 32 + (lane & 31);
#pragma unroll
                for (int mb = 0; mb < kPkMB; ++mb) {
                    if (mb >= nmb) break;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row = mb * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                        ep[row * kPkEpiStride] = f32_to_bf16_bits(swiglu<ACT>(acc[mb][0][r] + bg, acc[mb][1][r] + bu));
                    }
                }
            }
            __syncthreads();
            uint16_t* glu = reinterpret_cast<uint16_t*>(prm.out);
            const int col0 = wi.n_idx * kPkWaves * 32;
            for (int i = tid; i < rows * (kPkWaves * 4); i += kPkThreads) {
                const int row = i / (kPkWaves * 4), c = i % (kPkWaves * 4);
                const int col = col0 + 8 * c;
                if (col < prm.F)
                    *reinterpret_cast<u32x4*>(glu + (long long)(row_begin + row) * prm.F + col) =
                        *reinterpret_cast<const u32x4*>(s_epi + row * kPkEpiStride + 8 * c);
            }
        } else {
            if (!active) continue;
            float* Y = reinterpret_cast<float*>(prm.out);
            float bn[2] = {0.f, 0.f};
            if constexpr (HAS_BIAS) {
#pragma unroll
                for (int f = 0; f < 2; ++f) bn[f] = prm.bias[(long long)e * prm.H + 64 * g + 32 * f + (lane & 31)];
            }
#pragma unroll
            for (int mb = 0; mb < kPkMB; ++mb) {
                if (mb >= nmb) break;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = mb * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (row < rows) {
                        const int p = s_pair[row];
                        const float w = s_w[row];
#pragma unroll
                        for (int f = 0; f < 2; ++f)
                            Y[(long long)p * prm.H + 64 * g + 32 * f + (lane & 31)] = (acc[mb][f][r] + bn[f]) * w;
                    }
                }
            }
        }
    }
}

static int g_pk_cu_count = 0;

static int pk_cu_count() {
    if (g_pk_cu_count == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            g_pk_cu_count = n;
        else
            g_pk_cu_count = 256;
    }
    return g_pk_cu_count;
}

template <int MODE, int ACT, bool HAS_BIAS>
static hipError_t launch_pk_t(const PkParams& prm, int max_tiles, hipStream_t s) {
    int grid = min(max_tiles * prm.n_tiles, pk_cu_count());
    grid = ceil_div(max(grid, 1), 8) * 8;
    hipLaunchKernelGGL((moe_gemm_packed_kernel<MODE, ACT, HAS_BIAS>), dim3(grid), dim3(kPkThreads), 0, s, prm);
    return hipGetLastError();
}

hipError_t launch_route(const int32_t* idx, int T, int K, int E, int BM, int32_t* offsets, int32_t* sorted_pairs,
                        int32_t* tile_offsets, int32_t* tile_expert, int32_t* meta, int32_t* counts,
                        hipStream_t stream);
hipError_t launch_combine(const float* Y, const int32_t* idx, uint16_t* out, int T, int K, int E, int H,
                          hipStream_t s);

int packed_tile_m() { return kPkBM; }

// route -> packed gate_up GEMM -> packed down GEMM -> combine, all on stream s. Shapes were checked
// by the caller (H % 64 == 0, F % 64 == 0, E <= 1024, T >= 1).
hipError_t launch_prefill_packed(const void* x, const void* w1p, const float* b1, const void* w2p, const float* b2,
                                 const int32_t* idx, const float* route_w, int T, int H, int F, int E, int K,
                                 int bias_interleaved, int act, void* out, int32_t* offsets, int32_t* tile_offsets,
                                 int32_t* meta, int32_t* sorted_pairs, int32_t* tile_expert, int32_t* route_counts,
                                 int max_tiles, uint16_t* glu, float* Y, hipStream_t s, hipEvent_t* ev) {
    auto mark = [&](int i) { if (ev) (void)hipEventRecord(ev[i], s); };
    mark(0);
    hipError_t st =
        launch_route(idx, T, K, E, kPkBM, offsets, sorted_pairs, tile_offsets, tile_expert, meta, route_counts, s);
    if (st != hipSuccess) return st;
    mark(1);
    PkParams g1{};
    g1.A = static_cast<const uint16_t*>(x);
    g1.B = static_cast<const uint16_t*>(w1p);
    g1.bias = b1;
    g1.sorted_pairs = sorted_pairs;
    g1.offsets = offsets;
    g1.tile_offsets = tile_offsets;
    g1.tile_expert = tile_expert;
    g1.meta = meta;
    g1.route_w = route_w;
    g1.out = glu;
    g1.Kd = H;
    g1.NG = F / 32;
    g1.KS = H / 16;
    g1.n_tiles = ceil_div(g1.NG, kPkWaves);
    g1.F = F;
    g1.H = H;
    g1.topk = K;
    g1.bias_interleaved = bias_interleaved;
    if (act == kActSilu)
        st = b1 ? launch_pk_t<kModePkGateUp, kActSilu, true>(g1, max_tiles, s)
                : launch_pk_t<kModePkGateUp, kActSilu, false>(g1, max_tiles, s);
    else
        st = b1 ? launch_pk_t<kModePkGateUp, kActGptOss, true>(g1, max_tiles, s)
                : launch_pk_t<kModePkGateUp, kActGptOss, false>(g1, max_tiles, s);
    if (st != hipSuccess) return st;
    mark(2);
    PkParams g2 = g1;
    g2.A = glu;
    g2.B = static_cast<const uint16_t*>(w2p);
    g2.bias = b2;
    g2.out = Y;
    g2.Kd = F;
    g2.NG = H / 64;
    g2.KS = F / 16;
    g2.n_tiles = ceil_div(g2.NG, kPkWaves);
    st = b2 ? launch_pk_t<kModePkDown, kActSilu, true>(g2, max_tiles, s)
            : launch_pk_t<kModePkDown, kActSilu, false>(g2, max_tiles, s);
    if (st != hipSuccess) return st;
    mark(3);
    st = launch_combine(Y, idx, static_cast<uint16_t*>(out), T, K, E, H, s);
    mark(4);
    return st;
}

}  // namespace cmoe
