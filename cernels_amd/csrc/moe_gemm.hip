// Prefill grouped GEMMs for the routed experts, bf16 MFMA on gfx950.
//
//   GEMM1  glu[r, :]  = act( X[tok(r), :] · W1_e^T )   rows r of expert e, SwiGLU in the epilogue
//   GEMM2  Y[p, :]    = w_p · ( glu[r, :] · W2_e^T + b2_e )   24-bit floats, at the pair's own row p
//   combine out[t, :] = bf16( sum_k Y[t*K + k, :] )   (slots in k order; moe_combine_h_kernel)
// Y keeps 16 mantissa bits: rounding each of the K weighted rows to bf16 before the k-sum costs about
// 0.006*RMS of extra error, more than the 2e-2*RMS budget leaves after the output's own rounding.
//
// glu as a bf16 pair. GEMM1 stores each glu value v as hi = bf16(v) and lo = bf16(v - hi); hi + lo
// carries v to about 2^-17 relative, where one bf16 rounding (2^-9) costs up to 0.008*RMS of output
// error (0.0207 / 0.0226 / 0.0262 against the 2e-2*RMS bar on the deepseek-v2-lite, 30B-A3B and
// qwen3-next Zipf workloads, by a float64 simulation of that rounding alone; with the pair the error
// is the output's own bf16 rounding, 0.0127 / 0.0189 / 0.0183). A glu row is 2F bf16 values: per
// 64 columns, the 64 hi values then the 64 lo values. A GEMM2 stage holds both halves of one 64-wide
// k-chunk of glu beside that chunk's weights, and every weight fragment read from LDS feeds two MFMAs
// (hi, then lo): GEMM2's MFMAs double, its weight loads do not.
//
// Replaces the reference's per-expert host loop (src/kops/cohere2_moe_experts/csrc/
// cohere2_moe_experts.cu:315-358: gather_kernel, cublasGemmEx x2, swiglu_kernel,
// scatter_add_f32_kernel, final cast; gpt-oss adds add_gateup_bias_kernel,
// src/kops/gpt_oss_moe_experts/csrc/gpt_oss_moe_experts.cu:75-117). Here the gather is folded
// into GEMM1's operand load, the SwiGLU (and the gpt-oss gate_up bias) into GEMM1's epilogue,
// the down bias and routing weight into GEMM2's epilogue, and no host synchronisation is needed:
// the GEMMs read the tile list the route kernel left in device memory.
//
// Scheduling: a persistent grid (a multiple of 8 workgroups). Work items are (expert, N-tile,
// M-tile) in expert-major order, M fastest, so the M-tiles that share one weight tile are
// neighbours. Workgroup b runs on XCD b % 8; item range [x*per, (x+1)*per) is given to XCD x so
// that neighbours share that XCD's L2 and each weight tile is fetched from HBM about once.
//
// One tile kernel for both weight layouts (moe_gemm_v3_kernel: 128 x 256 tiles, 8 waves, both operands
// copied HBM -> LDS directly). The concat layout's weights are K-contiguous and are read like the
// activations; the interleaved gpt-oss layout's weights are N-contiguous and stay so in LDS, where
// ds_read_b64_tr_b16 hands each lane the 8 consecutive k of its column (b_frag_nc).
#include "moe_tile.h"

namespace cmoe {

constexpr int kBM = 128;  // rows of an M-tile (the route's tile list is built for it)

// Kernel modes.
constexpr int kModeGateUp = 0;
constexpr int kModeDown = 1;

struct GemmParams {
    const uint16_t* A;             // GEMM1: x [T, H]; GEMM2: glu pairs [P, 2F] (rows in expert order)
    const uint16_t* B;             // expert weights, expert 0
    const float* bias;             // GEMM1: [E, 2F]; GEMM2: [E, H]; or null
    const int32_t* sorted_pairs;   // [P] pair id per expert-ordered row
    const int32_t* offsets;        // [E+1]
    const int32_t* tile_offsets;   // [E+1]
    const int32_t* tile_expert;    // [tiles]
    const int32_t* meta;           // [0] = tiles
    const float* route_w;          // [P] fp32 routing weight per pair (GEMM2)
    void* out;                     // GEMM1: glu pairs bf16 [P, 2F]; GEMM2: Y fp32 [P, H]
    int Kdim;                      // A's row length: H (GEMM1) or 2F (GEMM2, the glu pairs)
    int N;                         // output columns: F (GEMM1) or H (GEMM2)
    int F;                         // expert intermediate size
    int topk;
    int n_tiles;                   // output column tiles
    long long expert_stride;       // elements of one expert's matrix in B
    int ldb;                       // row stride of B (elements)
};

// glu value v as the bf16 pair (hi, lo): hi = bf16(v), lo = bf16(v - hi) (lo = 0 where v is not finite).
__device__ __forceinline__ void split_bf16(float v, uint16_t& hi, uint16_t& lo) {
    hi = f32_to_bf16_bits(v);
    const float r = v - bf16_bits_to_f32(hi);
    lo = f32_to_bf16_bits(r == r && fabsf(r) != __builtin_inff() ? r : 0.f);
}

// Offset of glu column n's hi value in a glu row of the pair layout (its lo value is 64 further).
__device__ __forceinline__ int glu_pair_col(int n) { return 128 * (n >> 6) + (n & 63); }

// ---- grouped GEMM: 128 x 256 tiles, 8 waves, direct-to-LDS pipeline ------------------------------
//
// Both operands stream HBM -> LDS with global_load_lds_dwordx4: the activations (and concat weights,
// K-contiguous [rows, K]) in the swizzled row layout of lds_off, interleaved weights ([K, N]) in the
// N-contiguous layout of nc_off. GEMM1 keeps three 48 KB stages (two in flight while the oldest is
// consumed); a GEMM2 stage holds the hi and the lo tile of one 64-wide glu chunk beside its weight tile
// (64 KB), two stages deep. 512 threads = 8 waves = two per SIMD, arranged 2 (M) x 4 (N); each wave owns
// a 64 x 64 block of v_mfma_f32_32x32x16_bf16 results.
//   GEMM1 (gate_up), concat: the 256 B-rows are 128 gate rows then the 128 matching up rows, so a
//     wave's two 32-column blocks are the gate and the up value of the same 32 glu columns.
//   GEMM1, interleaved: the 256 B-columns are 128 (gate, up) column pairs as stored; a lane holds a
//     gate and its neighbour lane the matching up, paired in the epilogue by a lane exchange.
//   GEMM2 (down): the 256 B-rows (concat) or B-columns (interleaved) are 256 consecutive output columns.
// Epilogue: the accumulators go through LDS (the pipeline buffers are free by then) so that every
// row leaves as contiguous stores: 2 x 256 B of bf16 glu (hi, lo) per row, 768 B of 24-bit Y per output
// row (12 bytes per four columns).
constexpr int kV3BM = 128;
constexpr int kV3BN = 256;
constexpr int kV3Threads = 512;
constexpr int kV3Waves = kV3Threads / kWave;
constexpr int kV3ABytes = kV3BM * kBK * 2;         // 16 KB
constexpr int kV3BBytes = kV3BN * kBK * 2;         // 32 KB
constexpr int kV3APer = kV3BM / 8 / kV3Waves;      // 1 KB copies per wave per stage: A 2 (or 4: hi, lo), B 4
constexpr int kV3BPer = kV3BN / 8 / kV3Waves;
// GEMM1: three stages of A 16 KB + B 32 KB; GEMM2: two stages of A hi 16 KB + A lo 16 KB + B 32 KB
template <int MODE> constexpr int v3_stages() { return MODE == kModeDown ? 2 : 3; }
template <int MODE> constexpr int v3_a_tiles() { return MODE == kModeDown ? 2 : 1; }
template <int MODE> constexpr int v3_stage_bytes() { return v3_a_tiles<MODE>() * kV3ABytes + kV3BBytes; }
constexpr int kV3Lds = 3 * (kV3ABytes + kV3BBytes);  // 144 KB (GEMM2 uses 128)
static_assert(2 * (2 * kV3ABytes + kV3BBytes) <= kV3Lds, "GEMM2 stages fit the allocation");
constexpr int kV3YStride = kV3BN + 4;              // fp32 epilogue row stride (bank offset per row)
constexpr int kV3GStride = kV3BN / 2 + 8;          // bf16 epilogue row stride

// The B tile of the interleaved layout keeps the weights' own [K][N] order (N-contiguous rows of 256
// columns, 512 bytes); 16-byte chunk q of k-row r sits at chunk q ^ (4 (r % 4)), so the four k-rows and
// four chunks one half-wave's transposed reads touch fall on distinct banks.
__device__ __forceinline__ int nc_off(int row, int col) {
    return row * (kV3BN * 2) + (((col >> 3) ^ (4 * (row & 3))) << 4) + ((col & 7) << 1);
}

// B operand of v_mfma_f32_32x32x16_bf16 (lane l: k = kb + 8 (l / 32) + 0..7, column cb + l % 32) from an
// N-contiguous tile, by two ds_read_b64_tr_b16. Within each 16-lane group the lanes' 8-byte rows form a
// 16 x 4 matrix S of 16-bit values and lane i receives S[4r + i/4][i%4], r = 0..3; so lane i' of a group
// reading row k0 + i'/4 at column c0 + 4 (i' % 4) receives k-rows k0..k0+3 of column c0 + i'.
__device__ __forceinline__ bf16x8 b_frag_nc(const unsigned char* sB, int kb, int cb, int lane) {
    typedef short v4i16 __attribute__((ext_vector_type(4)));
    const int g = lane >> 4, i = lane & 15;
    const int row = kb + 8 * (g >> 1) + (i >> 2), col = cb + 16 * (g & 1) + 4 * (i & 3);
    auto rd = [&](int r) {
        return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16*)(lds_u32(sB) + nc_off(r, col)));
    };
    const v4i16 lo = rd(row), hi = rd(row + 4);
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

template <int MODE, int LAYOUT, int ACT, bool HAS_BIAS>
__global__ __launch_bounds__(kV3Threads, 1) void moe_gemm_v3_kernel(GemmParams prm) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    constexpr bool kNc = LAYOUT == kLayoutInterleaved;  // weights N-contiguous: B tile [64 k][256 n]
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int wm = wave & 1, wn = wave >> 1;
    const uint32_t lds0 = lds_u32(smem);
    const int lrow = lane >> 3;

    const int tiles = prm.meta[0];
    const int total = tiles * prm.n_tiles;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, slots = gridDim.x >> 3;
    const int per = ceil_div(total, 8);
    const int it_end = min(total, (xcd + 1) * per);
    const int halfN = kV3BN / 2;

    for (int it = xcd * per + slot; it < it_end; it += slots) {
        const int e = prm.tile_expert[it / prm.n_tiles];
        const int t0 = prm.tile_offsets[e], nt_e = prm.tile_offsets[e + 1] - t0;
        const int local = it - t0 * prm.n_tiles;
        const int n_idx = local / nt_e, m_idx = local - n_idx * nt_e;
        const int seg0 = prm.offsets[e], seg_n = prm.offsets[e + 1] - seg0;
        int row_begin, rows;  // the expert's M-tiles split its rows evenly in 32-row blocks
        tile_rows(m_idx, nt_e, seg_n, row_begin, rows);
        row_begin += seg0;
        const int n0 = n_idx * (MODE == kModeGateUp ? halfN : kV3BN);  // first output column
        const uint16_t* Be = prm.B + (long long)e * prm.expert_stride;
        const int Kd = prm.Kdim;

        const uint16_t* a_src[kV3APer];
        const uint16_t* b_src[kV3BPer];
#pragma unroll
        for (int i = 0; i < kV3APer; ++i) {
            const int r = 8 * (i * kV3Waves + wave) + lrow;
            const int ra = min(r, rows - 1);
            long long src_row;
            if constexpr (MODE == kModeGateUp) src_row = prm.sorted_pairs[row_begin + ra] / prm.topk;
            else src_row = row_begin + ra;
            a_src[i] = prm.A + src_row * Kd + ((lane & 7) ^ swz(r)) * 8;
        }
#pragma unroll
        for (int i = 0; i < kV3BPer; ++i) {
            if constexpr (kNc) {
                // copy i of this wave: k-rows 2c and 2c+1 (c = i*8 + wave), 32 chunks of 8 columns each; the chunk
                // a lane writes (its LDS position) is loaded from chunk position ^ 4 (row % 4); columns past the
                // matrix read a valid column (their results are not stored)
                const int r = 2 * (i * kV3Waves + wave) + (lane >> 5);
                const int ncols = MODE == kModeGateUp ? 2 * prm.F : prm.N;
                const int c0 = MODE == kModeGateUp ? 2 * n0 : n0;
                const int col = min(c0 + 8 * ((lane & 31) ^ (4 * (r & 3))), ncols - 8);
                b_src[i] = Be + (long long)r * prm.ldb + col;
            } else {
                const int r = 8 * (i * kV3Waves + wave) + lrow;
                int wrow;
                if constexpr (MODE == kModeGateUp) {
                    const int c = min(n0 + (r & (halfN - 1)), prm.F - 1);
                    wrow = r < halfN ? c : prm.F + c;
                } else {
                    wrow = min(n0 + r, prm.N - 1);
                }
                b_src[i] = Be + (long long)wrow * prm.ldb + ((lane & 7) ^ swz(r)) * 8;
            }
        }
        constexpr int S = v3_stages<MODE>(), AT = v3_a_tiles<MODE>(), SB = v3_stage_bytes<MODE>();
        constexpr int kCopies = AT * kV3APer + kV3BPer;  // copies per wave per stage
        auto issue = [&](int kt, int stage) {
            const uint32_t sa = lds0 + stage * SB + wave * 1024;
#pragma unroll
            for (int h = 0; h < AT; ++h)  // GEMM2: A columns [128 kt, 128 kt + 64) hi, then the lo half
#pragma unroll
                for (int i = 0; i < kV3APer; ++i)
                    dma16(a_src[i] + kt * AT * kBK + h * kBK, sa + h * kV3ABytes + i * (kV3Waves * 1024));
#pragma unroll
            for (int i = 0; i < kV3BPer; ++i)
                dma16(b_src[i] + (kNc ? (long long)kt * kBK * prm.ldb : (long long)kt * kBK),
                      sa + AT * kV3ABytes + i * (kV3Waves * 1024));
        };

        f32x16 acc[2][2];
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

        // the wave's two 32-column blocks: B-tile rows (concat) or columns (interleaved; for gate_up 32 physical
        // columns are 16 gate/up pairs)
        int brow[2];
        if constexpr (MODE == kModeGateUp && !kNc) {
            brow[0] = wn * 32;
            brow[1] = halfN + wn * 32;
        } else {
            brow[0] = wn * 64;
            brow[1] = wn * 64 + 32;
        }
        const int arow0 = wm * 64 + (lane & 31);
        const int khalf = lane >> 5;
        const int nk = Kd / (AT * kBK);  // GEMM2: Kd = 2F, one stage per 64-wide k-chunk of glu

        wait_vmcnt<0>();  // index loads above must not be counted against the copies below
#pragma unroll
        for (int s = 0; s < S - 1; ++s)
            if (s < nk) issue(s, s);
        for (int kt = 0; kt < nk; ++kt) {
            if constexpr (S == 3) {
                if (kt + 1 < nk) wait_vmcnt<kCopies>();  // stage kt+1 may stay in flight
                else wait_vmcnt<0>();
            } else {
                wait_vmcnt<0>();  // two stages: stage kt+1 is issued after the barrier below
            }
            __syncthreads();
            if (kt + S - 1 < nk) issue(kt + S - 1, (kt + S - 1) % S);
            const unsigned char* sA = smem + (kt % S) * SB;
            const unsigned char* sB = sA + AT * kV3ABytes;
            bf16x8 af[kBK / 16][2][AT], bfr[kBK / 16][2];
#pragma unroll
            for (int ks = 0; ks < kBK / 16; ++ks) {
                const int chunk = ks * 2 + khalf;
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int h = 0; h < AT; ++h)
                        af[ks][mb][h] =
                            *reinterpret_cast<const bf16x8*>(sA + h * kV3ABytes + lds_off(arow0 + mb * 32, chunk));
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    if constexpr (kNc) bfr[ks][nb] = b_frag_nc(sB, 16 * ks, brow[nb], lane);
                    else bfr[ks][nb] = *reinterpret_cast<const bf16x8*>(sB + lds_off(brow[nb] + (lane & 31), chunk));
                }
            }
#pragma unroll
            for (int ks = 0; ks < kBK / 16; ++ks)
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                        for (int h = 0; h < AT; ++h)
                            acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks][mb][h], bfr[ks][nb],
                                                                                  acc[mb][nb], 0, 0, 0);
        }
        __syncthreads();  // all waves are done reading the pipeline buffers; reuse them for the epilogue

        // ---- epilogue through LDS. Accumulator element r of a 32x32 block sits at
        // row 8*(r/4) + 4*(lane/32) + (r%4), column lane & 31.
        if constexpr (MODE == kModeGateUp) {
            uint16_t* stg = reinterpret_cast<uint16_t*>(smem);  // [2][128][kV3GStride]: the hi tile, the lo tile
            if constexpr (kNc) {
                // physical column 2j is gate, 2j + 1 up of glu column j: even lanes hold gates, their odd
                // neighbours the matching ups
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    const int pc = brow[nb] + (lane & 31);          // physical column within the tile
                    const int c = (brow[nb] >> 1) + ((lane & 31) >> 1);  // glu column within the tile
                    float b = 0.f;
                    if constexpr (HAS_BIAS) b = prm.bias[(long long)e * 2 * prm.F + min(2 * n0 + pc, 2 * prm.F - 1)];
#pragma unroll
                    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const float v = acc[mb][nb][r] + b;
                            const float u = __shfl_xor(v, 1, kWave);
                            if (!(lane & 1)) {
                                const int row = wm * 64 + mb * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                                uint16_t hi, lo;
                                split_bf16(swiglu<ACT>(v, u), hi, lo);
                                stg[row * kV3GStride + c] = hi;
                                stg[(kV3BM + row) * kV3GStride + c] = lo;
                            }
                        }
                }
            } else {
                const int c = wn * 32 + (lane & 31);  // glu column within the tile
                float bg = 0.f, bu = 0.f;
                if constexpr (HAS_BIAS) {
                    const int n = min(n0 + c, prm.F - 1);
                    bg = prm.bias[(long long)e * 2 * prm.F + n];
                    bu = prm.bias[(long long)e * 2 * prm.F + prm.F + n];
                }
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row = wm * 64 + mb * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                        uint16_t hi, lo;
                        split_bf16(swiglu<ACT>(acc[mb][0][r] + bg, acc[mb][1][r] + bu), hi, lo);
                        stg[row * kV3GStride + c] = hi;
                        stg[(kV3BM + row) * kV3GStride + c] = lo;
                    }
            }
            __syncthreads();
            uint16_t* glu = reinterpret_cast<uint16_t*>(prm.out);
            constexpr int kChunks = kV3BN / 2 / 8;  // 16-byte chunks per glu row and half (16)
            for (int i = tid; i < kV3BM * 2 * kChunks; i += kV3Threads) {
                const int row = i / (2 * kChunks), rem = i - row * (2 * kChunks);
                const int half = rem / kChunks, ch = rem - half * kChunks;  // half 0: hi, 1: lo
                const int n = n0 + ch * 8;
                if (row < rows && n < prm.N)
                    *reinterpret_cast<u32x4*>(glu + (long long)(row_begin + row) * 2 * prm.F + glu_pair_col(n) +
                                              64 * half) =
                        *reinterpret_cast<const u32x4*>(stg + (half * kV3BM + row) * kV3GStride + ch * 8);
            }
        } else {
            float* stg = reinterpret_cast<float*>(smem);  // [128][kV3YStride] fp32 tile
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row = wm * 64 + mb * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                        stg[row * kV3YStride + brow[nb] + (lane & 31)] = acc[mb][nb][r];
                    }
            __syncthreads();
            // Y rows in the 24-bit float form (four columns per 12 bytes): the combine sums the K rows of a
            // token from values rounded at 2^-16, at 3/4 of fp32's bytes
            unsigned char* Yb = reinterpret_cast<unsigned char*>(prm.out);
            constexpr int kChunks = kV3BN / 4;  // four-column groups per output row (64)
            for (int i = tid; i < kV3BM * kChunks; i += kV3Threads) {
                const int row = i / kChunks, ch = i - row * kChunks;
                const int n = n0 + ch * 4;
                if (row < rows && n < prm.N) {
                    const int p = prm.sorted_pairs[row_begin + row];
                    const float w = prm.route_w[p];
                    f32x4 v = *reinterpret_cast<const f32x4*>(stg + row * kV3YStride + ch * 4);
                    if constexpr (HAS_BIAS) {
                        const f32x4 b = *reinterpret_cast<const f32x4*>(prm.bias + (long long)e * prm.N + n);
                        v += b;
                    }
                    v *= w;
                    const f24x4 q = pack_f24x4(v[0], v[1], v[2], v[3]);
                    __builtin_memcpy(Yb + ((long long)p * prm.N + n) * 3, &q, 12);
                }
            }
        }
        __syncthreads();  // the staging tile is reused by the next item's copies
    }
}


static int g_cu_count = 0;

static int cu_count() {
    if (g_cu_count == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            g_cu_count = n;
        else
            g_cu_count = 256;
    }
    return g_cu_count;
}

int gemm_tile_m() { return kBM; }

template <int MODE, int LAYOUT, int ACT, bool HAS_BIAS>
static hipError_t launch_v3_t(const GemmParams& prm, int upper, hipStream_t stream) {
    static bool attr = false;
    if (!attr) {
        hipError_t st = hipFuncSetAttribute((const void*)moe_gemm_v3_kernel<MODE, LAYOUT, ACT, HAS_BIAS>,
                                            hipFuncAttributeMaxDynamicSharedMemorySize, kV3Lds);
        if (st != hipSuccess) return st;
        attr = true;
    }
    int grid = min(upper, cu_count());
    grid = ceil_div(max(grid, 1), 8) * 8;
    hipLaunchKernelGGL((moe_gemm_v3_kernel<MODE, LAYOUT, ACT, HAS_BIAS>), dim3(grid), dim3(kV3Threads), kV3Lds,
                       stream, prm);
    return hipGetLastError();
}

template <int MODE, int LAYOUT, int ACT, bool HAS_BIAS>
static hipError_t launch_gemm_t(const GemmParams& prm, int max_tiles, hipStream_t stream) {
    return launch_v3_t<MODE, LAYOUT, ACT, HAS_BIAS>(prm, max_tiles * prm.n_tiles, stream);
}

hipError_t launch_gateup(const GemmParams& prm, int layout, int act, bool has_bias, int max_tiles, hipStream_t s) {
    if (layout == kLayoutConcat) {
        if (act == kActSilu)
            return has_bias ? launch_gemm_t<kModeGateUp, kLayoutConcat, kActSilu, true>(prm, max_tiles, s)
                            : launch_gemm_t<kModeGateUp, kLayoutConcat, kActSilu, false>(prm, max_tiles, s);
        return has_bias ? launch_gemm_t<kModeGateUp, kLayoutConcat, kActGptOss, true>(prm, max_tiles, s)
                        : launch_gemm_t<kModeGateUp, kLayoutConcat, kActGptOss, false>(prm, max_tiles, s);
    }
    if (act == kActSilu)
        return has_bias ? launch_gemm_t<kModeGateUp, kLayoutInterleaved, kActSilu, true>(prm, max_tiles, s)
                        : launch_gemm_t<kModeGateUp, kLayoutInterleaved, kActSilu, false>(prm, max_tiles, s);
    return has_bias ? launch_gemm_t<kModeGateUp, kLayoutInterleaved, kActGptOss, true>(prm, max_tiles, s)
                    : launch_gemm_t<kModeGateUp, kLayoutInterleaved, kActGptOss, false>(prm, max_tiles, s);
}

hipError_t launch_down(const GemmParams& prm, int layout, bool has_bias, int max_tiles, hipStream_t s) {
    if (layout == kLayoutConcat)
        return has_bias ? launch_gemm_t<kModeDown, kLayoutConcat, kActSilu, true>(prm, max_tiles, s)
                        : launch_gemm_t<kModeDown, kLayoutConcat, kActSilu, false>(prm, max_tiles, s);
    return has_bias ? launch_gemm_t<kModeDown, kLayoutInterleaved, kActSilu, true>(prm, max_tiles, s)
                    : launch_gemm_t<kModeDown, kLayoutInterleaved, kActSilu, false>(prm, max_tiles, s);
}

hipError_t launch_combine_h(const unsigned char* Y, const int32_t* idx, uint16_t* out, int T, int K, int E, int H,
                            const int32_t* sync, const int8_t* psig, const float* b2, const float* route_w,
                            hipStream_t s);

hipError_t launch_route(const int32_t* idx, int T, int K, int E, int BM, int32_t* offsets, int32_t* sorted_pairs,
                        int32_t* tile_offsets, int32_t* tile_expert, int32_t* meta, int32_t* counts,
                        int32_t* sched, hipStream_t stream, int8_t* row_zero = nullptr,
                        const XcdSplit* split = nullptr);

// route -> gate_up GEMM -> down GEMM -> combine, all on stream s. Shapes were checked by the caller
// (H % 64 == 0, F % 64 == 0, E <= 1024, T >= 1).
hipError_t launch_prefill(const void* x, const void* w1, const float* b1, const void* w2, const float* b2,
                          const int32_t* idx, const float* route_w, int T, int H, int F, int E, int K, int layout,
                          int act, void* out, int32_t* offsets, int32_t* tile_offsets, int32_t* meta,
                          int32_t* sorted_pairs, int32_t* tile_expert, int32_t* route_counts, int max_tiles,
                          uint16_t* glu, float* Y, hipStream_t s, hipEvent_t* ev) {
    // ev (optional): 5 events recorded before route, after route, after gate_up, after down,
    // after combine — for per-stage timing on the caller's stream.
    auto mark = [&](int i) { if (ev) (void)hipEventRecord(ev[i], s); };
    mark(0);
    hipError_t st =
        launch_route(idx, T, K, E, kBM, offsets, sorted_pairs, tile_offsets, tile_expert, meta, route_counts, nullptr, s);
    if (st != hipSuccess) return st;
    mark(1);
    const bool concat = layout == kLayoutConcat;
    GemmParams g1{};
    g1.A = static_cast<const uint16_t*>(x);
    g1.B = static_cast<const uint16_t*>(w1);
    g1.bias = b1;
    g1.sorted_pairs = sorted_pairs;
    g1.offsets = offsets;
    g1.tile_offsets = tile_offsets;
    g1.tile_expert = tile_expert;
    g1.meta = meta;
    g1.route_w = route_w;
    g1.out = glu;
    g1.Kdim = H;
    g1.N = F;
    g1.F = F;
    g1.topk = K;
    g1.n_tiles = ceil_div(F, kV3BN / 2);
    g1.expert_stride = 2LL * F * H;
    g1.ldb = concat ? H : 2 * F;
    st = launch_gateup(g1, layout, act, b1 != nullptr, max_tiles, s);
    if (st != hipSuccess) return st;
    mark(2);
    GemmParams g2 = g1;
    g2.A = glu;
    g2.B = static_cast<const uint16_t*>(w2);
    g2.bias = b2;
    g2.out = Y;
    g2.Kdim = 2 * F;  // the glu pair: 2F bf16 values per row
    g2.N = H;
    g2.n_tiles = ceil_div(H, kV3BN);
    g2.expert_stride = (long long)H * F;
    g2.ldb = concat ? F : H;
    st = launch_down(g2, layout, b2 != nullptr, max_tiles, s);
    if (st != hipSuccess) return st;
    mark(3);
    // Y already holds w (glu W2 + b2): the combine adds no bias and reads no glu scale
    st = launch_combine_h(reinterpret_cast<const unsigned char*>(Y), idx, static_cast<uint16_t*>(out), T, K, E, H,
                          nullptr, nullptr, nullptr, route_w, s);
    mark(4);
    return st;
}

}  // namespace cmoe
