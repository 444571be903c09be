// Prefill grouped GEMMs over expert weights packed in MFMA-fragment order (bf16 MFMA, gfx950).
//
// Same mathematics as the grouped GEMMs on the transformers layouts (moe_gemm.hip):
//   GEMM1  glu[r, :] = act( X[tok(r), :] · W1_e + b1_e )        SwiGLU / gpt-oss gate in the epilogue
//   GEMM2  Y[p, :]   = w_p · ( glu[r, :] · W2_e + b2_e )        routing weight in the epilogue (fp32)
// and the same route kernel, item list and deterministic k-sum combine. What changes is how the
// weights reach the matrix cores. The weights are re-laid once (cernels_moe_pack_weights) so that
// each 32x16 MFMA operand fragment is 1 KB of contiguous memory in exactly the order a wave's lanes
// consume it. A wave streams its weight columns straight into registers with one contiguous 1 KB
// read per fragment: nothing of the weights goes through LDS. Only the activation tile (token rows
// gathered through the expert-sorted pair list) is staged in LDS, where all eight waves of the
// workgroup read it.
//
// Workgroup: 8 waves (two per SIMD), one workgroup per CU, items of 256 rows x 8 fragments. Each
// wave owns one 32-column weight fragment for all 256 rows of the item (eight 32x32 accumulator
// blocks), so a weight fragment is fetched once per item and feeds 8 MFMAs, and the activation tile
// is fetched once per item and feeds 8 fragments. The CU's vector-memory pipe (address and data
// units, L1) carries 8 KB per 32 MFMAs of a wave, which is what bounds this kernel at these shapes,
// not HBM. Blocks past the item's rows are skipped (the k-loop is instantiated per block count).
// K advances in stages of 64: weight loads are issued two stages, activation loads one stage
// before their MFMAs.
//
// GEMM1 fragments hold 16 gate and the 16 matching up columns, so one wave holds both inputs of the
// gated activation for its 16 glu columns; a v_permlane16_swap pairs them up in the epilogue.
#include <type_traits>

#include "moe_tile.h"

namespace cmoe {

constexpr int kPkWaves = 8;                 // waves per workgroup = fragments per N-tile
constexpr int kPkThreads = kPkWaves * kWave;
constexpr int kPkBM = 256;
constexpr int kPkMB = kPkBM / 32;           // 32-row MFMA blocks per item
constexpr int kPkABytes = kPkBM * kBK * 2;  // 32 KB A stage
constexpr int kPkFrag = 512;                // bf16 elements of one fragment (1 KB)
constexpr int kPkGlu = kPkWaves * 16;       // glu columns of a GEMM1 N-tile
constexpr int kPkEpiStride = kPkGlu + 8;    // bf16 row stride of the GEMM1 output tile in LDS
constexpr int kPkBDepth = 2;                // weight stages held in registers per wave

constexpr int kModePkGateUp = 0;
constexpr int kModePkDown = 1;

// Packed layout of one projection, viewed as B[k][n] (reduction length Kd, KS = Kd/16 k-steps) cut
// into NF fragments of 32 columns:
//   gate_up: fragment c = gate columns [16c, 16c+16) then up columns [16c, 16c+16). Kd = H, NF = F/16.
//   down:    fragment c = output columns [32c, 32c+32).                           Kd = F, NF = H/32.
// Fragments are bundled by eight (an N-tile: one fragment per wave) and stored k-step-major inside a
// tile, so the eight waves of a workgroup read one contiguous 8 KB run per k-step. Lane l of
// fragment (c, ks) holds B[16ks + 8(l/32) + j][column l%32 of the fragment], j = 0..7.
// Returns the fragment's index in 1 KB units.
__host__ __device__ inline long long packed_frag(int e, int c, int ks, int NF, int KS) {
    const int t = c >> 3, w = c & 7, nw = min(8, NF - 8 * t);
    return (long long)e * NF * KS + 8LL * KS * t + (long long)ks * nw + w;
}

// ---- packing (one-time, per weight tensor) ---------------------------------------------------------
// One thread per 16-byte lane chunk of the packed output, in logical (e, c, ks, lane) order.
template <int WHICH, int LAYOUT>
__global__ __launch_bounds__(256) void moe_pack_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                       int E, int H, int F) {
    const int Kd = WHICH == 0 ? H : F;
    const int NF = WHICH == 0 ? F / 16 : H / 32;
    const int KS = Kd / 16;
    const long long total = (long long)E * NF * KS * kWave;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int lane = (int)(i % kWave);
    long long q = i / kWave;
    const int ks = (int)(q % KS);
    q /= KS;
    const int c = (int)(q % NF);
    const int e = (int)(q / NF);
    const int k0 = 16 * ks + 8 * (lane >> 5);
    const int col = lane & 31;
    u32x4 v;
    if constexpr (WHICH == 0) {
        const int f = col >> 4;                // 0 = gate, 1 = up
        const int fc = 16 * c + (col & 15);    // intermediate index
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
        const int n = 32 * c + col;  // output (hidden) index
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
    *reinterpret_cast<u32x4*>(dst + packed_frag(e, c, ks, NF, KS) * kPkFrag + lane * 8) = v;
}

size_t packed_weight_bytes(int H, int F, int E, int which) {
    (void)which;  // both projections keep their element count: 2FH (gate_up) and HF (down)
    return which == 0 ? (size_t)E * 2 * F * H * 2 : (size_t)E * H * F * 2;
}

hipError_t launch_pack(const uint16_t* src, uint16_t* dst, int E, int H, int F, int layout, int which, hipStream_t s) {
    const long long chunks = (long long)E * (which == 0 ? 2LL * F * H : (long long)H * F) / 8;  // = E*NF*KS*64
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
    int Kd, NF, KS, n_tiles;
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
        const int fc = wi.n_idx * kPkWaves + wave;
        const int nmb = ceil_div(rows, 32);  // non-empty 32-row blocks
        const bool active = fc < prm.NF;     // wave-uniform: this wave stores results

        __syncthreads();  // the previous item is done with the LDS buffers and the pair table
        if constexpr (MODE == kModePkDown) {
            if (tid < rows) {
                const int p = prm.sorted_pairs[row_begin + tid];
                s_pair[tid] = p;
                s_w[tid] = prm.route_w[p];
            }
        }
        // A rows: thread t loads 16-byte chunk t%8 of rows t/8 + 64i of each stage; a wave instruction
        // covers 8 rows x 128 B. Rows past the item's end re-read its last row.
        const int a_chunk = tid & 7;
        const uint16_t* a_src[kPkMB / 2];
#pragma unroll
        for (int i = 0; i < kPkMB / 2; ++i) {
            const int ra = min((tid >> 3) + 64 * i, rows - 1);
            long long src_row;
            if constexpr (MODE == kModePkGateUp) src_row = prm.sorted_pairs[row_begin + ra] / prm.topk;
            else src_row = row_begin + ra;
            a_src[i] = prm.A + src_row * Kd + a_chunk * 8;
        }
        const int fcc = active ? fc : wi.n_idx * kPkWaves;  // idle waves read the tile's first fragment
        const int nw = min(kPkWaves, prm.NF - kPkWaves * wi.n_idx);
        const uint16_t* b_ptr = prm.B + packed_frag(e, fcc, 0, prm.NF, prm.KS) * kPkFrag + lane * 8;
        const long long b_step = (long long)nw * kPkFrag;  // elements between consecutive k-steps

        f32x16 acc[kPkMB];
#pragma unroll
        for (int mb = 0; mb < kPkMB; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mb][r] = 0.f;

        // Activation chunks are loaded at the start of the step before their MFMAs and written to
        // LDS at its end. Weight fragments sit in kPkBDepth register slots of four k-steps; k-step q
        // of slot d is refilled with the stage kPkBDepth ahead as soon as its MFMAs have read it.
        // Every load is visible to the compiler, which waits for exactly the loads each use needs.
        // Loads and MFMAs are never behind a branch, so those waits stay exact and the loop is one
        // basic block: past the last stage a step re-reads the last stage (an L2 hit), and a wave
        // whose fragment is past the end (only in a projection's last N-tile) computes on valid
        // fragments of the tile and stores nothing.
        auto kloop = [&](auto nc) {
            constexpr int NMB = decltype(nc)::value;  // 32-row blocks computed
            constexpr int NA = (NMB + 1) / 2;         // activation chunks per thread per stage
            u32x4 areg[NA];
            u32x4 breg[kPkBDepth][4];
            auto load_a = [&](int s) {
                const int sc = min(s, nst - 1);
#pragma unroll
                for (int i = 0; i < NA; ++i) areg[i] = *reinterpret_cast<const u32x4*>(a_src[i] + sc * kBK);
            };
            auto load_b = [&](int s, auto dc, int q) {  // k-step q of stage s into slot d
                constexpr int d = decltype(dc)::value;
                const uint16_t* bp = b_ptr + (long long)(4 * min(s, nst - 1) + q) * b_step;
                breg[d][q] = *reinterpret_cast<const u32x4*>(bp);
            };
            auto store_a = [&](auto bc) {  // the loaded activation chunks -> LDS buffer b
                constexpr int b = decltype(bc)::value;
                unsigned char* sA = smem + b * kPkABytes;
#pragma unroll
                for (int i = 0; i < NA; ++i)
                    *reinterpret_cast<u32x4*>(sA + lds_off((tid >> 3) + 64 * i, a_chunk)) = areg[i];
            };
            // One A fragment register per 32-row block: right after block mb's MFMA at k-step q
            // consumes it, it is reloaded with block mb's fragment of k-step q + 1, which then has
            // the other blocks' MFMAs to arrive. The weight loads of the stage kPkBDepth ahead are
            // spread over the four k-steps (fenced with sched_barrier) so that the CU's address
            // unit works on them while the matrix cores run.
            auto step = [&](int s, auto bc, auto dc) {
                constexpr int b = decltype(bc)::value;
                constexpr int d = decltype(dc)::value;
                __syncthreads();  // stage s is in LDS buffer b; every wave is done with the other buffer
                const unsigned char* sA = smem + b * kPkABytes;
                auto read_af = [&](int q, int mb) {
                    return *reinterpret_cast<const bf16x8*>(sA + lds_off(mb * 32 + (lane & 31), 2 * q + (lane >> 5)));
                };
                load_a(s + 1);  // mostly L2 hits: arrive within this step's MFMAs
                bf16x8 af[NMB];
#pragma unroll
                for (int mb = 0; mb < NMB; ++mb) af[mb] = read_af(0, mb);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    __builtin_amdgcn_sched_barrier(0);
                    const bf16x8 bq = __builtin_bit_cast(bf16x8, breg[d][q]);
#pragma unroll
                    for (int mb = 0; mb < NMB; ++mb) {
                        acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mb], bq, acc[mb], 0, 0, 0);
                        if (q + 1 < 4) af[mb] = read_af(q + 1, mb);
                    }
                    load_b(s + kPkBDepth, dc, q);  // the registers just consumed
                    // Keep the order written above: MFMA, then the LDS read that refills its A
                    // register, block by block; then the weight load.
#pragma unroll
                    for (int mb = 0; mb < NMB; ++mb) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                // MFMA
                        if (q + 1 < 4) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                    }
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
                }
                __builtin_amdgcn_sched_barrier(0);
                store_a(IC<1 - b>{});  // stage s+1's chunks -> the other LDS buffer
            };
            load_a(0);
#pragma unroll
            for (int q = 0; q < 4; ++q) load_b(0, IC<0>{}, q);
#pragma unroll
            for (int q = 0; q < 4; ++q) load_b(1, IC<1>{}, q);
            store_a(IC<0>{});
            int s = 0;
            for (; s + 1 < nst; s += 2) {
                step(s, IC<0>{}, IC<0>{});
                step(s + 1, IC<1>{}, IC<1>{});
            }
            if (s < nst) step(s, IC<0>{}, IC<0>{});
        };
        static_assert(kPkBDepth == 2, "the k-loop above alternates two weight slots");
        switch (nmb) {
            case 1: kloop(IC<1>{}); break;
            case 2: kloop(IC<2>{}); break;
            case 3: kloop(IC<3>{}); break;
            case 4: kloop(IC<4>{}); break;
            case 5: kloop(IC<5>{}); break;
            case 6: kloop(IC<6>{}); break;
            case 7: kloop(IC<7>{}); break;
            default: kloop(IC<8>{}); break;
        }

        // ---- epilogue. Element r of a 32x32 accumulator block is at row 8*(r/4) + 4*(lane/32) + (r%4),
        // column lane & 31.
        if constexpr (MODE == kModePkGateUp) {
            // Columns 0-15 of the fragment are gate, 16-31 the matching up columns. v_permlane16_swap
            // exchanges lanes 16-31 (48-63) of accumulator element r with lanes 0-15 (32-47) of
            // element r+4 (8 rows further down): afterwards every lane holds gate and up of one
            // (row, glu column), with rows r in lanes 0-15 and 32-47 and rows r+4 in the others.
            // The bf16 tile is staged in LDS, then written as 16-byte chunks: each output row of the
            // N-tile is one contiguous 256-byte run.
            if (active) {
                const int fcol = 16 * fc + (lane & 15);
                float bg = 0.f, bu = 0.f;
                if constexpr (HAS_BIAS) {
                    const float* be = prm.bias + (long long)e * 2 * prm.F;
                    bg = prm.bias_interleaved ? be[2 * fcol] : be[fcol];
                    bu = prm.bias_interleaved ? be[2 * fcol + 1] : be[prm.F + fcol];
                }
                uint16_t* ep = s_epi + wave * 16 + (lane & 15);
                const int rlane = 4 * (lane >> 5) + 8 * ((lane >> 4) & 1);
#pragma unroll
                for (int mb = 0; mb < kPkMB; ++mb) {
                    if (mb >= nmb) break;
#pragma unroll
                    for (int h = 0; h < 2; ++h)
#pragma unroll
                        for (int r4 = 0; r4 < 4; ++r4) {
                            const int r = 8 * h + r4;
                            // __float_as_uint takes the element by value (a bit_cast of an ext-vector
                            // element lvalue reads element 0 with this compiler).
                            const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(acc[mb][r]),
                                                                             __float_as_uint(acc[mb][r + 4]), false, false);
                            const float gate = __uint_as_float(sw[0]);
                            const float up = __uint_as_float(sw[1]);
                            const int row = mb * 32 + 16 * h + r4 + rlane;
                            ep[row * kPkEpiStride] = f32_to_bf16_bits(swiglu<ACT>(gate + bg, up + bu));
                        }
                }
            }
            __syncthreads();
            uint16_t* glu = reinterpret_cast<uint16_t*>(prm.out);
            const int col0 = wi.n_idx * kPkGlu;
            for (int i = tid; i < rows * (kPkGlu / 8); i += kPkThreads) {
                const int row = i / (kPkGlu / 8), c = i % (kPkGlu / 8);
                const int col = col0 + 8 * c;
                if (col < prm.F)
                    *reinterpret_cast<u32x4*>(glu + (long long)(row_begin + row) * prm.F + col) =
                        *reinterpret_cast<const u32x4*>(s_epi + row * kPkEpiStride + 8 * c);
            }
        } else {
            if (!active) continue;
            float* Y = reinterpret_cast<float*>(prm.out);
            const int n = 32 * fc + (lane & 31);
            float bn = 0.f;
            if constexpr (HAS_BIAS) bn = prm.bias[(long long)e * prm.H + n];
#pragma unroll
            for (int mb = 0; mb < kPkMB; ++mb) {
                if (mb >= nmb) break;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = mb * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (row < rows) Y[(long long)s_pair[row] * prm.H + n] = (acc[mb][r] + bn) * s_w[row];
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
    int grid = min(max_tiles * prm.n_tiles, pk_cu_count());  // one workgroup per CU
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
    g1.NF = F / 16;
    g1.KS = H / 16;
    g1.n_tiles = ceil_div(g1.NF, kPkWaves);
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
    g2.NF = H / 32;
    g2.KS = F / 16;
    g2.n_tiles = ceil_div(g2.NF, kPkWaves);
    st = b2 ? launch_pk_t<kModePkDown, kActSilu, true>(g2, max_tiles, s)
            : launch_pk_t<kModePkDown, kActSilu, false>(g2, max_tiles, s);
    if (st != hipSuccess) return st;
    mark(3);
    st = launch_combine(Y, idx, static_cast<uint16_t*>(out), T, K, E, H, s);
    mark(4);
    return st;
}

}  // namespace cmoe
