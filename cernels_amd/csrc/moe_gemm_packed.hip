// Prefill grouped GEMMs over expert weights packed in MFMA-fragment order (bf16 MFMA, gfx950).
//
// Same mathematics as the grouped GEMMs on the transformers layouts (moe_gemm.hip):
//   GEMM1  glu[r, :] = act( X[tok(r), :] · W1_e + b1_e )        SwiGLU / gpt-oss gate in the epilogue
//   GEMM2  Y[p, :]   = w_p · ( glu[r, :] · W2_e )                routing weight in the epilogue (fp32)
//   combine out[t, :] = sum_k Y[t*K + k, :] + w_p · b2_e            down bias with the k-sum
// and the same route kernel, item list and deterministic k-sum combine. What changes is how the
// weights reach the matrix cores. The weights are re-laid once (cernels_moe_pack_weights) so that
// each 32x16 MFMA operand fragment is 1 KB of contiguous memory in exactly the order a wave's lanes
// consume it. A wave streams its weight columns straight into registers with one contiguous 1 KB
// read per fragment: nothing of the weights goes through LDS. Only the activation tile (token rows
// gathered through the expert-sorted pair list) goes to LDS, copied there directly from global memory
// (buffer_load ... lds, no registers), where all eight waves of the workgroup read it.
//
// Workgroup: 8 waves (two per SIMD), one workgroup per CU, items of 256 rows x 8 fragments. Each
// wave owns one 32-column weight fragment for all 256 rows of the item (eight 32x32 accumulator
// blocks), so a weight fragment is fetched once per item and feeds 8 MFMAs, and the activation tile
// is fetched once per item and feeds 8 fragments. The CU's vector-memory pipe (address and data
// units, L1) carries 8 KB per 32 MFMAs of a wave, and with it the L2 misses of the weight stream,
// which is what bounds this kernel at these shapes. Blocks past the item's rows are skipped (the
// k-loop is instantiated per block count). K advances in stages of 64 held in three LDS buffers and
// three weight register slots: both operands of a stage are requested two stages before its MFMAs.
//
// GEMM1 fragments hold 16 gate and the 16 matching up columns, so one wave holds both inputs of the
// gated activation for its 16 glu columns: elements r and r + 8 of a lane's accumulator block are gate
// and up of the same glu column, and the activation runs in registers. In both epilogues lanes l and
// l + 32 hold alternate groups of four columns of one row; a v_permlane32_swap per dword trades groups
// between the half-waves so that each lane stores one contiguous run with 16-byte stores.
//
// Precision of the second projection. glu (the activation output, GEMM2's A operand) is stored as
// fp16, not bf16: 2^-11 relative rounding instead of 2^-8, which is what keeps the output within
// 2e-2*RMS of the exact value (a bf16 glu alone costs up to ~0.008*RMS). The down weights are packed
// as fp16 too (MFMA operands share one type), each 32-column fragment scaled by a power of two so its
// largest |w| sits in [2^14, 2^15): the conversion from bf16 is exact there, and the epilogue
// multiplies the fragment's columns back by that power of two. A glu segment (a row's 16 or 32
// columns of one GEMM1 wave) whose largest |glu| m reaches 2^15 is stored scaled by 2^-s (s >= 1, so it
// cannot overflow fp16), and so is a segment with 0 < m < 2^-8 (s <= -23: scaled up, so its values do
// not fall into fp16's subnormals, whose fixed 2^-24 spacing would leave small rows with a large
// relative error); both put m * 2^-s in [2^14, 2^15) and mark the row. An all-zero segment records
// kGluAnyScale (it is exact at every scale). A small kernel between the two GEMMs then brings every
// marked row to its segments' largest s and records it per pair; the combine multiplies that pair's
// row by 2^s. Without marked rows (the normal case) that kernel reads one flag and exits.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "moe_split.h"
#include "moe_tile.h"

namespace cmoe {

constexpr int kPkWaves = 8;                 // waves per workgroup = fragments per N-tile
constexpr int kPkThreads = kPkWaves * kWave;
constexpr int kPkBM = 256;
constexpr int kPkMB = kPkBM / 32;           // 32-row MFMA blocks per item
constexpr int kPkABytes = kPkBM * kBK * 2;  // 32 KB A stage
constexpr int kPkFrag = 512;                // bf16 elements of one fragment (1 KB)
constexpr int kPkGlu = kPkWaves * 16;       // glu columns of a GEMM1 N-tile
constexpr int kPkStages = 3;                // activation LDS buffers = weight register slots per wave
constexpr int kPkMaxTail = 16;              // most items split into halves at the end of an XCD's range
// Items split at the end of each XCD's range: 12 for gate_up where experts average fewer rows than one M-tile,
// none otherwise and none for down. A half item keeps its full item's weight stream for half the MFMA work, so
// the split pays only where item costs are uneven. Measured in one process against no split (two alternations,
// gate_up µs per launch): Zipf (80 rows per expert) 241.3/245.5 -> 235.3/233.3; gpt-oss (512 rows per expert, whose
// M-tiles split its rows evenly) 502.8/502.6 -> 512.5/510.1 (16 items: within a few µs of 12); down with 8 or
// 12 items: equal or up to 12 µs slower on gpt-oss.
constexpr int kPkTailGateUp = 12;
// glu segments: scaled up below this largest |glu| (2^-8), down at or above 2^15; an all-zero segment
// records kGluAnyScale in gexp
constexpr float kGluSmall = 0.00390625f;
constexpr int kGluAnyScale = -128;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kModePkGateUp = 0;
constexpr int kModePkDown = 1;
constexpr int kModePkUp = 2;  // non-gated first projection (megablocks): glu[r, :] = act(X[tok(r), :] · W1_e)

// Packed layout of one projection, viewed as B[k][n] (reduction length Kd, KS = Kd/16 k-steps) cut
// into NF fragments of 32 columns:
//   gate_up: fragment c = gate columns [16c, 16c+16) then up columns [16c, 16c+16). Kd = H, NF = F/16.
//   down:    fragment c = output columns [32c, 32c+32).                           Kd = F, NF = H/32.
//   up:      (non-gated) fragment c = columns [32c, 32c+32), packed as a down projection with H and F
//            exchanged.                                                           Kd = H, NF = F/32.
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
// WHICH 0: gate_up (bf16). WHICH 1: down or the non-gated first projection. For down, `exps` holds
// the per-(expert, fragment) power of two of each 32-column fragment and the chunk is converted to
// fp16 scaled by it; for the non-gated first projection `exps` is null and the chunk stays bf16.
template <int WHICH, int LAYOUT>
__global__ __launch_bounds__(256) void moe_pack_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                       int E, int H, int F, const int8_t* __restrict__ exps) {
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
        if (exps) {  // bf16 -> fp16 * 2^-s: exact while the scaled value is a normal fp16
            const int sc = -(int)exps[(long long)e * NF + c];
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = pack_f16x2(__builtin_amdgcn_ldexpf(bf16_lo(v[j]), sc),
                                                          __builtin_amdgcn_ldexpf(bf16_hi(v[j]), sc));
        }
    }
    *reinterpret_cast<u32x4*>(dst + packed_frag(e, c, ks, NF, KS) * kPkFrag + lane * 8) = v;
}

// Power of two of each 32-column fragment of a down projection: s with max|w| * 2^-s in [2^14, 2^15)
// (0 for an all-zero fragment). One workgroup per (expert, fragment); the fragment is 32 output rows of
// [E, H, F] (contiguous) or 32 output columns of [E, F, H].
template <int LAYOUT>
__global__ __launch_bounds__(256) void moe_pack_exp_kernel(const uint16_t* __restrict__ src, int8_t* __restrict__ exps,
                                                           int H, int F) {
    const int NF = H / 32;
    const int e = blockIdx.x / NF, c = blockIdx.x - e * NF;
    float m = 0.f;
    if constexpr (LAYOUT == kLayoutConcat) {
        const u32x4* p = reinterpret_cast<const u32x4*>(src + ((long long)e * H + 32 * c) * F);
        for (int i = threadIdx.x; i < 32 * F / 8; i += blockDim.x) {
            const u32x4 v = p[i];
#pragma unroll
            for (int j = 0; j < 4; ++j) m = fmaxf(m, fmaxf(fabsf(bf16_lo(v[j])), fabsf(bf16_hi(v[j]))));
        }
    } else {
        for (int i = threadIdx.x; i < F * 4; i += blockDim.x) {  // row k, 16-byte chunk i % 4 of the 32 columns
            const u32x4 v = *reinterpret_cast<const u32x4*>(src + ((long long)e * F + i / 4) * H + 32 * c + 8 * (i % 4));
#pragma unroll
            for (int j = 0; j < 4; ++j) m = fmaxf(m, fmaxf(fabsf(bf16_lo(v[j])), fabsf(bf16_hi(v[j]))));
        }
    }
    m = wave_max(m);
    __shared__ float part[4];
    if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        const float mm = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
        exps[blockIdx.x] = (int8_t)(mm > 0.f ? max(-100, min(100, __builtin_amdgcn_frexp_expf(mm) - 15)) : 0);
    }
}

// Bytes of the per-(expert, fragment) exponent table that follows the packed down weights.
static size_t down_exp_bytes(int H, int E) { return ((size_t)E * (H / 32) + 255) / 256 * 256; }

size_t packed_weight_bytes(int H, int F, int E, int which) {
    // gate_up: 2FH bf16; down: HF fp16 + the exponent table; non-gated first projection: HF bf16
    if (which == 0) return (size_t)E * 2 * F * H * 2;
    return (size_t)E * H * F * 2 + (which == 1 ? down_exp_bytes(H, E) : 0);
}

hipError_t launch_pack(const uint16_t* src, uint16_t* dst, int E, int H, int F, int layout, int which, hipStream_t s) {
    if (which == 0) {
        const long long chunks = (long long)E * 2LL * F * H / 8;  // = E*NF*KS*64
        const unsigned grid = (unsigned)((chunks + 255) / 256);
        if (layout == kLayoutConcat) hipLaunchKernelGGL((moe_pack_kernel<0, kLayoutConcat>), dim3(grid), dim3(256), 0, s, src, dst, E, H, F, nullptr);
        else hipLaunchKernelGGL((moe_pack_kernel<0, kLayoutInterleaved>), dim3(grid), dim3(256), 0, s, src, dst, E, H, F, nullptr);
        return hipGetLastError();
    }
    // up ([E, F, H] concat = rows are outputs, or [E, H, F] interleaved = k-major) is a down projection
    // with H and F exchanged, kept in bf16 (its A operand is x)
    const int Hd = which == 2 ? F : H, Fd = which == 2 ? H : F;
    int8_t* exps = nullptr;
    if (which == 1) {
        exps = reinterpret_cast<int8_t*>(dst + (long long)E * H * F);
        const unsigned g = (unsigned)(E * (H / 32));
        if (layout == kLayoutConcat) hipLaunchKernelGGL((moe_pack_exp_kernel<kLayoutConcat>), dim3(g), dim3(256), 0, s, src, exps, H, F);
        else hipLaunchKernelGGL((moe_pack_exp_kernel<kLayoutInterleaved>), dim3(g), dim3(256), 0, s, src, exps, H, F);
    }
    const long long chunks = (long long)E * Hd * Fd / 8;
    const unsigned grid = (unsigned)((chunks + 255) / 256);
    if (layout == kLayoutConcat) hipLaunchKernelGGL((moe_pack_kernel<1, kLayoutConcat>), dim3(grid), dim3(256), 0, s, src, dst, E, Hd, Fd, exps);
    else hipLaunchKernelGGL((moe_pack_kernel<1, kLayoutInterleaved>), dim3(grid), dim3(256), 0, s, src, dst, E, Hd, Fd, exps);
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
    const int32_t* bounds;         // [9] per-XCD item ranges written by the route, or null: equal split
    const float* route_w;          // [P] (GEMM2)
    void* out;                     // GEMM1: glu fp16 [P, F]; GEMM2: Y as 24-bit floats [P, H]
    int Kd, NF, KS, n_tiles;
    int F, H, topk;
    int bias_interleaved;          // GEMM1 bias order: 0 = [gate F | up F], 1 = gate/up interleaved
    int a_bytes;                   // GEMM1: bytes of x (< 2^31, checked by the caller)
    int fw;                        // fragments per item (<= kPkWaves); waves past fw idle
    int* counters;                 // [8] per-XCD work counters, zeroed by the route kernel
    int8_t* gexp;                  // GEMM1: [F/16, p_cap] exponent of each 16-column glu row segment
                                   // (kGluAnyScale: all zero)
    int8_t* rsig;                  // [P] per glu row: 0, or (GEMM1) 1 = has a scaled segment, then its scale
    int32_t* sync;                 // [2]: [1] = "some glu segment is scaled"; zeroed by the route kernel
    int p_cap;                     // row stride of gexp (T*K)
    const int8_t* wexp;            // GEMM2: [E, NF] power of two of each packed fp16 weight fragment
    int tail;                      // items at the end of an XCD's range handed out as two halves (<= kPkMaxTail)
};


template <int N>
using IC = std::integral_constant<int, N>;

// MODE/ACT/HAS_BIAS select the projection; XPF: the reduction has at least two stages, and the
// next item's first two stages are copied and loaded during the current item's last two steps
// (cross-item prefetch); R3: the number of stages mod 3, which sets the k-loop's empty positions;
// PEEL (R3 == 2, at least 5 stages): the loop's last round of three steps runs after it.
template <int MODE, int ACT, bool HAS_BIAS, bool XPF, int R3, bool PEEL>
__global__ __launch_bounds__(kPkThreads, 1) void moe_gemm_packed_kernel(PkParams prm) {
    static_assert(XPF || R3 == 1, "without prefetch the reduction is one stage");
    static_assert(!PEEL || R3 == 2, "peeled only where no ordinary step follows the loop");
    static_assert(MODE != kModePkUp || !HAS_BIAS, "the non-gated projection has no bias");
    static_assert(MODE != kModePkDown || !HAS_BIAS, "the down bias is added by the combine");
    // GEMM2 multiplies fp16 glu by fp16 weights; the first projections bf16 x by bf16 weights.
    using OpT = std::conditional_t<MODE == kModePkDown, f16x8, bf16x8>;
    // the first projection gathers token rows of x through the pair list; down reads its own glu rows
    constexpr bool kGather = MODE != kModePkDown;
    // The activation stages: three LDS buffers, declared as separate arrays so that the compiler tells
    // a copy into one from a read of another (its wait before a read then covers only the copies into
    // that buffer).
    __shared__ __attribute__((aligned(16))) unsigned char sA0[kPkABytes];
    __shared__ __attribute__((aligned(16))) unsigned char sA1[kPkABytes];
    __shared__ __attribute__((aligned(16))) unsigned char sA2[kPkABytes];
    // Epilogue tables, double-buffered by item parity: row -> pair and routing weight (GEMM2), and
    // the N-tile's bias (GEMM1: 128 gate then 128 up entries; GEMM2: 256 columns).
    __shared__ int s_pair[2][kPkBM];
    __shared__ float s_w[2][kPkBM];
    __shared__ __attribute__((aligned(16))) float s_bias[2][2 * kPkGlu];
    // GEMM2: power of two of each wave's weight fragment (entry t holds fragment t % 8: every table
    // thread stores one, which keeps the table store free of a branch of its own)
    __shared__ int s_wx[2][kPkBM];
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);

    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, slots = gridDim.x >> 3;
    int b_lo, b_hi;
    if (prm.bounds) {
        b_lo = prm.bounds[xcd];
        b_hi = prm.bounds[xcd + 1];
    } else {
        const int total = prm.meta[0] * prm.n_tiles, per = ceil_div(total, 8);
        b_lo = min(xcd * per, total);
        b_hi = min(b_lo + per, total);
    }
    const int Kd = prm.Kd, nst = Kd / kBK;
    // A copy instruction puts lane l's 16 bytes at LDS position l of the wave's 1 KB (8 rows of the
    // tile), i.e. at chunk position tid & 7 of its row; in the swizzled layout (lds_off) that position
    // holds chunk (tid & 7) ^ swz(row), and swz(row) = (tid >> 4) & 7 for every row the thread copies.
    const int a_chunk = (tid & 7) ^ ((tid >> 4) & 7);

    // Items of XCD x are one contiguous range of the list, [bounds[x], bounds[x+1]) (moe_split.h: of
    // about equal estimated cost where workgroups run many items, else equal in count), so that the items that share
    // a weight tile (neighbours in the list) run at about the same time on one XCD's L2. Each slot of
    // the XCD takes offsets s and 2*slots-1-s first (snake order: long and short items mix on every CU), then draws
    // offsets 2*slots + n from the XCD's work counter: workgroups that run faster take more items,
    // so the launch does not end on the slowest workgroup's fixed share. (Drawing from the other
    // XCDs' counters once the own one is exhausted was measured slower: the blocking draws and the
    // lost L2 sharing cost more than the balance gained.)
    //
    // The tail: where an XCD's range holds at least three rounds of items, those of its last prm.tail items
    // that have more than 3/4 kPkBM rows are handed out as two halves (rows [0, kPkBM/2) and the rest), so
    // that the launch ends on shorter items. (Splitting items of fewer rows leaves a second half that costs
    // nearly a whole item: 30B-A3B's gate_up, ~130-160 rows per expert, went from 181 to 200 µs.) Every row is
    // still computed by one workgroup with the same k-loop, so the output is the same bit for bit. Work codes:
    // 4 * item + h, h = 0 whole, 1 first half, 2 second half; offsets past the whole items index the tail
    // table, built once per workgroup.
    const int n_items = b_hi - b_lo;
    const int n_tail = tail_items(n_items, slots, prm.tail, kPkMaxTail);
    const int n_whole = n_items - n_tail;  // >= 2 * slots, so the first two offsets never need the table
    __shared__ int s_tail[2 * kPkMaxTail];
    __shared__ int s_ntail;
    auto item_at = [&](int code, WorkItem& w) {  // code: work code, or -1
        if (code < 0) return false;
        w = decode_item(code >> 2, prm.n_tiles, prm.tile_expert, prm.tile_offsets, prm.offsets);
        tail_part(code & 3, kPkBM, w.row_begin, w.rows);
        return true;
    };
    auto item_of_off = [&](int off) {  // work code at offset off of this XCD's work, or -1
        if (off < n_whole) return 4 * (b_lo + off);
        if (n_tail == 0) return -1;
        const int t = off - n_whole;
        return __builtin_amdgcn_readfirstlane(t < s_ntail ? s_tail[t] : -1);  // uniform: a work code from LDS
    };
    __shared__ int s_next;  // work code of the item after next (or -1), published once per item
    // Operands are read with buffer loads: a 128-bit descriptor per operand and item (uniform,
    // SGPRs) plus a 32-bit per-lane offset, so the k-loop holds no 64-bit addresses.
    //   A: GEMM1 gathers token rows of x (descriptor over all of x); GEMM2 reads the item's own
    //      contiguous glu rows (descriptor at its first row). Thread t copies rows t/8 + 64i of the
    //      tile into LDS, clamped to the item's last row: a_row() is the row in the A matrix, a_off()
    //      its byte offset from the descriptor base (at the chunk this lane copies).
    //   B: the wave's fragment run from k-step 0; lane offset lane*16, k-step offsets uniform.
    auto a_row = [&](const WorkItem& w, int i) { return w.row_begin + min((tid >> 3) + 64 * i, w.rows - 1); };
    auto a_off = [&](const WorkItem& w, int src_row) {
        const int r = kGather ? src_row : src_row - w.row_begin;
        return (uint32_t)r * (uint32_t)(Kd * 2) + (uint32_t)a_chunk * 16u;
    };
    auto a_rsrc = [&](const WorkItem& w) {
        if constexpr (kGather)
            return __builtin_amdgcn_make_buffer_rsrc((void*)prm.A, (short)0, prm.a_bytes, kBufferWord3);
        else
            return __builtin_amdgcn_make_buffer_rsrc((void*)(prm.A + (long long)w.row_begin * Kd), (short)0,
                                                     w.rows * Kd * 2, kBufferWord3);
    };
    // This wave's fragment of an item; waves past the item's fragments (or past NF) are idle and
    // never load weights. Fragments are stored in bundles of eight, k-step-major inside a bundle.
    auto frag_of = [&](const WorkItem& w) { return min(w.n_idx * prm.fw + wave, prm.NF - 1); };
    auto b_rsrc = [&](const WorkItem& w) {
        const int fc = frag_of(w);
        const int nw = min(8, prm.NF - 8 * (fc >> 3));
        return __builtin_amdgcn_make_buffer_rsrc((void*)(prm.B + packed_frag(w.e, fc, 0, prm.NF, prm.KS) * kPkFrag),
                                                 (short)0, (prm.KS - 1) * nw * kPkFrag * 2 + 1024, kBufferWord3);
    };
    auto b_stride = [&](const WorkItem& w) { return min(8, prm.NF - 8 * (frag_of(w) >> 3)) * kPkFrag * 2; };
    // Table entries of an item for thread t (row t; bias entry t).
    auto tab_pair = [&](const WorkItem& w) { return prm.sorted_pairs[w.row_begin + min(tid, w.rows - 1)]; };
    auto tab_bias = [&](const WorkItem& w) {
        if constexpr (MODE == kModePkGateUp) {
            const int f = (tid >> 7) & 1, col = min(w.n_idx * 16 * prm.fw + (tid & (kPkGlu - 1)), prm.F - 1);
            const float* be = prm.bias + (long long)w.e * 2 * prm.F;
            return prm.bias_interleaved ? be[2 * col + f] : be[f * prm.F + col];
        } else {
            const int col = min(w.n_idx * 32 * prm.fw + (tid & (2 * kPkGlu - 1)), prm.H - 1);
            return prm.bias[(long long)w.e * prm.H + col];
        }
    };
    // GEMM2: the power of two of wave t's weight fragment.
    auto tab_wexp = [&](const WorkItem& w) {
        return (int)prm.wexp[(long long)w.e * prm.NF + min(w.n_idx * prm.fw + (tid & (kPkWaves - 1)), prm.NF - 1)];
    };
    // The row index is rebuilt here from the wave index (scalar) and the lane index (v_mbcnt, no inputs;
    // in asm, so that the compiler does not fold it back into the lane register it keeps): this store runs
    // at the end of the k-loop, where reloading a spilled lane register would wait for every load in flight.
    auto tab_store = [&](int buf, int pair, float w, float bias, int wx) {
        static_assert(kPkBM % kWave == 0, "the table rows are whole waves");
        if (wave < kPkBM / kWave) {
            int l;
            asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
            const int t = wave * kWave + l;
            if constexpr (MODE == kModePkDown) {
                s_pair[buf][t] = pair;
                s_w[buf][t] = w;
                s_wx[buf][t] = wx;
            }
            if constexpr (HAS_BIAS) s_bias[buf][t] = bias;
        }
    };

    WorkItem cur;
    if (!item_at(item_of_off(slot), cur)) return;
    int it_nx = item_of_off(2 * slots - 1 - slot);  // the next item
    // Thread 0 holds the counter ticket of the item after next: drawn one item ahead, so the
    // atomic's round trip is over long before its value is published.
    int ticket = 0;
    if (tid == 0) ticket = atomicAdd(prm.counters + xcd, 1);
    uint32_t a_cur[kPkMB / 2];  // activation row offsets of the current item
    __amdgpu_buffer_rsrc_t ra_cur = a_rsrc(cur), rb_cur = b_rsrc(cur);
    int bstep_cur = b_stride(cur);  // bytes between k-steps
    const uint32_t b_lane = (uint32_t)lane * 16u;

    f32x16 acc[kPkMB];
    static_assert(kPkStages == 3, "three LDS arrays below and the mod-3 step schedule of the k-loop");
    u32x4 breg[kPkStages][4];  // weight fragments: slot d holds the four k-steps of one stage
    auto sbuf = [&](auto bc) -> unsigned char* {
        constexpr int b = decltype(bc)::value;
        if constexpr (b == 0) return sA0;
        else if constexpr (b == 1) return sA1;
        else return sA2;
    };
    // The same buffer as an LDS-address-space pointer (the cast of the array itself folds away).
    using lds_bytes = __attribute__((address_space(3))) unsigned char*;
    auto sbuf_lds = [&](auto bc) { return (lds_bytes)sbuf(bc); };
    // Activation chunk i of this thread (tile row 64 i + tid / 8) of stage `stage`, copied from global
    // memory straight into LDS buffer b (no registers): 16 bytes per lane, the wave's 64 lanes fill the
    // 1 KB of rows 64 i + 8 wave .. 64 i + 8 wave + 7.
    auto copy_a = [&](__amdgpu_buffer_rsrc_t r, uint32_t ao, int stage, auto bc, int i) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            r, (__attribute__((address_space(3))) void*)(sbuf_lds(bc) + (64 * i + 8 * wave) * kBK * 2), 16, ao,
            stage * kBK * 2, 0, 0);
    };
    auto b_ld = [&](__amdgpu_buffer_rsrc_t r, int bs, int stage, int q) {
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, b_lane, (4 * stage + q) * bs, 0));
    };
    // Step barrier of a stage in buffer b. The read of buffer b makes the compiler wait for this wave's
    // copies into b (and only those: the buffers are separate arrays); after the barrier every wave's
    // copies into b have landed. There is no fence: a workgroup fence would wait for every copy in flight.
    auto stage_barrier = [&](auto bc) {
        asm volatile("" ::: "memory");
        const uint32_t v = *(volatile __attribute__((address_space(3))) const uint32_t*)sbuf_lds(bc);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        return v;  // consumed at the end of the step, so that its register is not reused (and waited for) early
    };
    // Barrier after LDS stores that other waves read (tables, the next work code): lgkmcnt(0) first.
    auto lds_barrier = [&]() {
        __builtin_amdgcn_s_waitcnt(0xC07F);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };
    // The whole set-up of one item without prefetch: offsets, tables into buffer tb, stages 0 and 1
    // (XPF) into LDS buffers and weight slots 0 and 1. Every wave has passed the previous item's last
    // barrier, so no wave still reads those buffers.
    auto start_item = [&](const WorkItem& w, int tb) {
        int pr[kPkMB / 2];
#pragma unroll
        for (int i = 0; i < kPkMB / 2; ++i) {
            if constexpr (kGather) pr[i] = prm.sorted_pairs[a_row(w, i)];
            else pr[i] = a_row(w, i);
        }
        int pair = 0, wx = 0;
        float rw = 0.f, bias = 0.f;
        if constexpr (MODE == kModePkDown) {
            pair = tab_pair(w);
            wx = tab_wexp(w);
        }
        if constexpr (HAS_BIAS) bias = tab_bias(w);
#pragma unroll
        for (int i = 0; i < kPkMB / 2; ++i)
            a_cur[i] = a_off(w, kGather ? pr[i] / prm.topk : pr[i]);
        if constexpr (MODE == kModePkDown) rw = prm.route_w[pair];
#pragma unroll
        for (int i = 0; i < kPkMB / 2; ++i) copy_a(ra_cur, a_cur[i], 0, IC<0>{}, i);
#pragma unroll
        for (int q = 0; q < 4; ++q) breg[0][q] = b_ld(rb_cur, bstep_cur, 0, q);
        if constexpr (XPF) {
#pragma unroll
            for (int i = 0; i < kPkMB / 2; ++i) copy_a(ra_cur, a_cur[i], 1, IC<1>{}, i);
#pragma unroll
            for (int q = 0; q < 4; ++q) breg[1][q] = b_ld(rb_cur, bstep_cur, 1, q);
        }
        tab_store(tb, pair, rw, bias, wx);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the tables are read after the first step's barrier
    };
    start_item(cur, 0);
    if (n_tail > 0 && wave == 0) {  // the tail table (read from the first item's end on; k-loop barriers order it)
        const int it = b_lo + n_whole + lane;
        bool split = false;
        if (lane < n_tail) {
            const WorkItem w = decode_item(it, prm.n_tiles, prm.tile_expert, prm.tile_offsets, prm.offsets);
            split = tail_splits(w.rows, kPkBM);
        }
        const uint64_t sb = __ballot(split);
        const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
        const int pos = lane + __popcll(sb & lt);
        if (lane < n_tail) {
            s_tail[pos] = 4 * it + (split ? 1 : 0);
            if (split) s_tail[pos + 1] = 4 * it + 2;
        }
        if (lane == 0) s_ntail = n_tail + __popcll(sb);
    }

    // One item; false once the work is done.
    auto item = [&](int j) -> bool {
        WorkItem nx;
        const bool has_nx = item_at(it_nx, nx);
        if (!has_nx) nx = cur;  // past the end the "next" loads re-read the current item
        const __amdgpu_buffer_rsrc_t ra_nx = a_rsrc(nx), rb_nx = b_rsrc(nx);
        const int bstep_nx = b_stride(nx);
        const int row_begin = cur.row_begin, rows = cur.rows;
        const int fc = cur.n_idx * prm.fw + wave;
        const bool active = wave < prm.fw && fc < prm.NF;  // wave-uniform
        const int nmb = ceil_div(rows, 32);  // non-empty 32-row blocks
        const int tb = j & 1;                // table buffer of this item
        // The next item's rows (GEMM1: their pair ids, loaded here, an item ahead of the copies that use them).
        int nxr[kPkMB / 2];
        if constexpr (XPF) {
#pragma unroll
            for (int i = 0; i < kPkMB / 2; ++i) {
                if constexpr (kGather) nxr[i] = prm.sorted_pairs[a_row(nx, i)];
                else nxr[i] = a_row(nx, i);
            }
        }
#pragma unroll
        for (int mb = 0; mb < kPkMB; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mb][r] = 0.f;

        // The k-loop runs over positions p = 0 .. NP-1, NP = nst rounded up to a multiple of 3: positions
        // below nst are the stages, the one or two above (if any) are empty. Position p uses LDS buffer and
        // weight register slot p % 3, so every item starts in buffer and slot 0 and its last two positions
        // are always in buffers 1 and 2. Step p runs the MFMAs of stage p, copies the activation rows of
        // stage p+2 into the buffer freed by step p-1 at its start and, k-step by k-step, loads the weights
        // of stage p+2 into the slot freed by step p-1: both operands arrive two steps ahead, and a step's
        // wait covers only its own stage. The last two positions load stages 0 and 1 of the next item
        // (XPF) instead, with its row offsets and tables, so the weights and activations keep streaming
        // through the epilogue (where the positions are empty, they have no MFMAs and the next item's
        // stages land during the epilogue). Loads and MFMAs are never behind a branch: the compiler's waits
        // stay exact and each step is one basic block.
        auto kloop = [&](auto nc) {
            constexpr int NMB = decltype(nc)::value;  // 32-row blocks computed; 0: idle wave
            // Activation chunks per thread per stage. The tile is shared: an idle wave still copies
            // its rows (all four chunks; rows past the item's blocks are never read).
            constexpr int NA = NMB > 0 ? (NMB + 1) / 2 : kPkMB / 2;
            int npair = 0, nwx = 0;
            float nbias = 0.f;
            // KIND 0: a stage, with the copies and weight loads of stage p + 2; 3: a stage whose p + 2 is
            // an empty position (no loads); 1: position NP-2 (next item's rows, stage 0, tables);
            // 2: position NP-1 (next item's stage 1, routing weights; all 256 rows of both stages).
            // EMPTY: a position past the last stage (no MFMAs).
            auto step = [&](int s, auto bc, auto kc, auto ec) {
                constexpr int b = decltype(bc)::value;
                constexpr int bn = (b + 2) % 3;  // buffer and slot of position p + 2
                constexpr int KIND = decltype(kc)::value;
                constexpr bool EMPTY = decltype(ec)::value;
                constexpr bool kNext = (KIND == 1 || KIND == 2) && XPF;  // loads for the next item
                constexpr bool kLoadW = KIND == 0 || kNext;
                const uint32_t probe = stage_barrier(IC<b>{});  // stage p is in LDS buffer b; buffer bn is free
                const unsigned char* sA = sbuf(IC<b>{});
                auto read_af = [&](int q, int mb) {
                    return *reinterpret_cast<const OpT*>(sA + lds_off(mb * 32 + (lane & 31), 2 * q + (lane >> 5)));
                };
                float nw = 0.f;
                if constexpr (KIND == 0) {
#pragma unroll
                    for (int i = 0; i < NA; ++i) copy_a(ra_cur, a_cur[i], s + 2, IC<bn>{}, i);
                } else if constexpr (kNext) {
                    if constexpr (KIND == 1) {
#pragma unroll
                        for (int i = 0; i < kPkMB / 2; ++i)
                            a_cur[i] = a_off(nx, kGather ? nxr[i] / prm.topk : nxr[i]);
                        if constexpr (MODE == kModePkDown) npair = tab_pair(nx);
                        if constexpr (HAS_BIAS) nbias = tab_bias(nx);
                    } else if constexpr (MODE == kModePkDown) {
                        nw = prm.route_w[npair];
                        nwx = tab_wexp(nx);
                    }
#pragma unroll
                    for (int i = 0; i < kPkMB / 2; ++i) copy_a(ra_nx, a_cur[i], KIND - 1, IC<bn>{}, i);
                }
                // A fragments in a ring of R registers: MFMA k (k-step k / NMB, block k % NMB) reads
                // slot k % R, which is then refilled with fragment k + R, R MFMAs ahead of its use.
                constexpr int R = NMB < 3 ? (NMB > 0 ? NMB : 1) : 3;
                constexpr int NK = 4 * NMB;
                OpT af[R];
                if constexpr (NMB > 0 && !EMPTY) {
#pragma unroll
                for (int k = 0; k < R; ++k) af[k] = read_af(k / NMB, k % NMB);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    // Raised wave priority for the k-step's MFMA group: while the other wave of the SIMD is
                    // in its step's non-MFMA part (first LDS reads, barrier), the wave that has MFMAs to
                    // issue wins the arbitration, which keeps the shared matrix unit fed.
                    __builtin_amdgcn_sched_barrier(0);
                    __builtin_amdgcn_s_setprio(1);
                    __builtin_amdgcn_sched_barrier(0);
                    const OpT bq = __builtin_bit_cast(OpT, breg[b][q]);
#pragma unroll
                    for (int mb = 0; mb < NMB; ++mb) {
                        const int k = q * NMB + mb;
                        // Weights as the first operand: the accumulator comes out transposed, each lane
                        // holding four consecutive output columns of one row.
                        if constexpr (MODE == kModePkDown)
                            acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bq, af[k % R], acc[mb], 0, 0, 0);
                        else
                            acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bq, af[k % R], acc[mb], 0, 0, 0);
                        if (k + R < NK) af[k % R] = read_af((k + R) / NMB, (k + R) % NMB);
                    }
                    if constexpr (KIND == 0) breg[bn][q] = b_ld(rb_cur, bstep_cur, s + 2, q);
                    else if constexpr (kNext) breg[bn][q] = b_ld(rb_nx, bstep_nx, KIND - 1, q);
                    // Keep the order written above: MFMA, then the LDS read that refills its A
                    // register, block by block; then the weight load.
#pragma unroll
                    for (int mb = 0; mb < NMB; ++mb) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                            // MFMA
                        if (q * NMB + mb + R < NK) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                    }
                    if (kLoadW) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
                    __builtin_amdgcn_sched_barrier(0);
                    __builtin_amdgcn_s_setprio(0);
                }
                } else if constexpr (kNext) {
                    // An idle wave may be active in the next item (and an empty position has no MFMAs): the
                    // next item's first two weight stages are loaded all the same.
#pragma unroll
                    for (int q = 0; q < 4; ++q) breg[bn][q] = b_ld(rb_nx, bstep_nx, KIND - 1, q);
                }
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (KIND == 2 && XPF) tab_store(tb ^ 1, npair, nw, nbias, nwx);
                asm volatile("" ::"v"(probe));
            };
            if constexpr (XPF) {
                // positions 0 .. nst-3 load stage p + 2: rounds of three, then L = (nst - 2) % 3 left over;
                // then E = NP - nst stages whose p + 2 is empty, then positions NP-2 and NP-1 (buffers 1, 2)
                constexpr int L = (R3 + 1) % 3, E = (3 - R3) % 3;
                const int M = nst - 2;
                int s = 0;
                // With no ordinary step between the loop and the last positions (L = 0), the compiler
                // reassigns the weight registers at the loop's exit and waits there for every load in flight;
                // running the loop's last round after it (PEEL) avoids that.
                for (; s + 3 + (PEEL ? 3 : 0) <= M; s += 3) {
                    step(s, IC<0>{}, IC<0>{}, IC<false>{});
                    step(s + 1, IC<1>{}, IC<0>{}, IC<false>{});
                    step(s + 2, IC<2>{}, IC<0>{}, IC<false>{});
                }
                if constexpr (PEEL) {
                    step(s, IC<0>{}, IC<0>{}, IC<false>{});
                    step(s + 1, IC<1>{}, IC<0>{}, IC<false>{});
                    step(s + 2, IC<2>{}, IC<0>{}, IC<false>{});
                    s += 3;
                }
                if constexpr (L >= 1) step(s, IC<0>{}, IC<0>{}, IC<false>{});
                if constexpr (L >= 2) step(s + 1, IC<1>{}, IC<0>{}, IC<false>{});
                if constexpr (E >= 1) step(nst - 2, IC<L % 3>{}, IC<3>{}, IC<false>{});
                if constexpr (E >= 2) step(nst - 1, IC<(L + 1) % 3>{}, IC<3>{}, IC<false>{});
                static_assert((L + E) % 3 == 1, "position NP-2 is in buffer 1");
                step(nst - 2 + E, IC<1>{}, IC<1>{}, IC<(E >= 2)>{});
                step(nst - 1 + E, IC<2>{}, IC<2>{}, IC<(E >= 1)>{});
            } else {
                step(0, IC<0>{}, IC<2>{}, IC<false>{});
            }
        };
        auto dispatch = [&]() {
            if (!active) {
                kloop(IC<0>{});
                return;
            }
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
        };
        dispatch();
        if (tid == 0) s_next = item_of_off(2 * slots + ticket);

        // ---- epilogue: element r of a transposed 32x32 accumulator block is row lane & 31 of the
        // block, column 8*(r/4) + 4*(lane/32) + (r%4) of the fragment. Only LDS reads and global
        // stores here: a global load would have to wait for the next item's weights in flight.
        if (active) {
            // lane & 31 and lane >> 5 rebuilt here from v_mbcnt (no inputs; in asm, so not hoisted): from the lane
            // register, the rows mb * 32 + (lane & 31) of all eight blocks were computed once before the item loop
            // and held through the k-loops or spilled (and then reloaded here behind the next item's loads).
            int lid;
            asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lid));
            const int lrow = lid & 31, half = lid >> 5;
            const int c4 = 4 * half;
            // glu stores: fp16 segments (16 columns per lane pair for gate_up, 32 for the non-gated
            // projection), each with its power of two s in gexp: 0, unless the segment's largest |glu| m
            // is 2^15 or more (or not finite) or below 2^-8 (and not 0); then the segment is stored
            // again, scaled by 2^-s. m = 0 records kGluAnyScale. fmaxf passes over nan values.
            uint16_t* glu = reinterpret_cast<uint16_t*>(prm.out);
            auto needs_scale = [](float m) { return !(m < 32768.f) || (m < kGluSmall && m > 0.f); };
            // s with m * 2^-s in [2^14, 2^15): s >= 1 for m >= 2^15 (inf or nan: s = 1), s <= -23 for
            // 0 < m < 2^-8 (clamped at -126, so 2^s stays a normal fp32 and s an int8 other than
            // kGluAnyScale)
            auto glu_scale = [](float m) {
                const int s = __builtin_amdgcn_frexp_expf(m) - 15;
                return m < 32768.f ? max(-126, s) : max(1, s);
            };
            auto mark_scaled = [&](long long r) {
                if (half == 0) prm.rsig[r] = 1;
                prm.sync[1] = 1;
            };
            if constexpr (MODE == kModePkGateUp) {
                // Fragment columns 0-15 are gate, 16-31 the matching up columns: elements r (< 8) and
                // r + 8 of one lane are gate and up of the same glu column.
                auto glu4 = [&](int mb, int i, float* v) {
                    f32x4 g4 = {0.f, 0.f, 0.f, 0.f}, u4 = {0.f, 0.f, 0.f, 0.f};
                    if constexpr (HAS_BIAS) {
                        g4 = *reinterpret_cast<const f32x4*>(&s_bias[tb][16 * wave + 8 * i + c4]);
                        u4 = *reinterpret_cast<const f32x4*>(&s_bias[tb][kPkGlu + 16 * wave + 8 * i + c4]);
                    }
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        float gv = acc[mb][4 * i + jj], uv = acc[mb][8 + 4 * i + jj];
                        if constexpr (HAS_BIAS) {  // x + 0.f is not folded (signed zero): add only a real bias
                            gv += g4[jj];
                            uv += u4[jj];
                        }
                        v[jj] = swiglu<ACT>(gv, uv);
                    }
                };
                // A lane holds glu columns c4 + 0..3 and c4 + 8..11 of the fragment's 16: one exchange between the
                // half-waves (columns 8-11 of lane l for 4-7 of lane l + 32) leaves lane l columns 0-7 and lane
                // l + 32 columns 8-15, one 16-byte store each. h: the two groups, two packed dwords each.
                auto store_glu = [&](uint16_t* g, uint32_t (&h)[4]) {
                    swap_halves(h[0], h[2]);
                    swap_halves(h[1], h[3]);
                    *reinterpret_cast<u32x4*>(g) = u32x4{h[0], h[1], h[2], h[3]};
                };
#pragma unroll
                for (int mb = 0; mb < kPkMB; ++mb) {
                    if (mb >= nmb) break;
                    const int row = mb * 32 + lrow;
                    if (row < rows) {  // lanes l and l ^ 32 hold the same row, so both run this or neither
                        const long long r = row_begin + row;
                        uint16_t* g = glu + r * prm.F + 16 * fc + 8 * half;
                        // the segment's largest |glu|; a nan is passed over (it reaches the output as a nan
                        // at any scale), an inf is not (scaled down, it keeps finite values finite)
                        float m = 0.f;
                        uint32_t h[4];
#pragma unroll
                        for (int i = 0; i < 2; ++i) {
                            float v[4];
                            glu4(mb, i, v);
#pragma unroll
                            for (int jj = 0; jj < 4; ++jj) m = fmaxf(m, fabsf(v[jj]));
                            h[2 * i] = pack_f16x2(v[0], v[1]);
                            h[2 * i + 1] = pack_f16x2(v[2], v[3]);
                        }
                        store_glu(g, h);
                        m = max_halves(m);  // the same on both lanes of the row
                        if (half == 0) prm.gexp[(long long)fc * prm.p_cap + r] = (int8_t)(m == 0.f ? kGluAnyScale : 0);
                        if (needs_scale(m)) {  // rare: the segment stored again, scaled, by the same lanes
                            const int sg = glu_scale(m);
#pragma unroll
                            for (int i = 0; i < 2; ++i) {
                                float v[4];
                                glu4(mb, i, v);
                                h[2 * i] = pack_f16x2(__builtin_amdgcn_ldexpf(v[0], -sg), __builtin_amdgcn_ldexpf(v[1], -sg));
                                h[2 * i + 1] = pack_f16x2(__builtin_amdgcn_ldexpf(v[2], -sg), __builtin_amdgcn_ldexpf(v[3], -sg));
                            }
                            store_glu(g, h);
                            if (half == 0) prm.gexp[(long long)fc * prm.p_cap + r] = (int8_t)sg;
                            mark_scaled(r);
                        }
                    }
                }
            } else if constexpr (MODE == kModePkUp) {
                // 16 columns of the fragment per lane (8i + c4 + jj), activation, fp16 glu row segment of
                // 32 columns (two gexp entries). Two exchanges between the half-waves (groups i = 0, 1 of lane
                // l + 32 for groups 2, 3 of lane l) leave lane l columns 0-15 and lane l + 32 columns 16-31, two
                // 16-byte stores each. s: the segment's scale (0: none).
                auto store_glu = [&](uint16_t* g, uint32_t (&h)[4][2]) {
#pragma unroll
                    for (int d = 0; d < 2; ++d) {
                        swap_halves(h[0][d], h[2][d]);
                        swap_halves(h[1][d], h[3][d]);
                    }
                    *reinterpret_cast<u32x4*>(g) = u32x4{h[0][0], h[0][1], h[2][0], h[2][1]};
                    *reinterpret_cast<u32x4*>(g + 8) = u32x4{h[1][0], h[1][1], h[3][0], h[3][1]};
                };
#pragma unroll
                for (int mb = 0; mb < kPkMB; ++mb) {
                    if (mb >= nmb) break;
                    const int row = mb * 32 + lrow;
                    if (row < rows) {  // lanes l and l ^ 32 hold the same row, so both run this or neither
                        const long long r = row_begin + row;
                        uint16_t* g = glu + r * prm.F + 32 * fc + 16 * half;
                        // the segment's largest |glu|; a nan is passed over (it reaches the output as a nan
                        // at any scale), an inf is not (scaled down, it keeps finite values finite)
                        float m = 0.f;
                        uint32_t h[4][2];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            float v[4];
#pragma unroll
                            for (int jj = 0; jj < 4; ++jj) {
                                v[jj] = act_plain<ACT>(acc[mb][4 * i + jj]);
                                m = fmaxf(m, fabsf(v[jj]));
                            }
                            h[i][0] = pack_f16x2(v[0], v[1]);
                            h[i][1] = pack_f16x2(v[2], v[3]);
                        }
                        store_glu(g, h);
                        m = max_halves(m);  // the same on both lanes of the row
                        if (half == 0) {
                            const int8_t s0 = (int8_t)(m == 0.f ? kGluAnyScale : 0);
                            prm.gexp[(long long)(2 * fc) * prm.p_cap + r] = s0;
                            prm.gexp[(long long)(2 * fc + 1) * prm.p_cap + r] = s0;
                        }
                        if (needs_scale(m)) {  // rare: the segment stored again, scaled, by the same lanes
                            const int sg = glu_scale(m);
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                float v[4];
#pragma unroll
                                for (int jj = 0; jj < 4; ++jj)
                                    v[jj] = __builtin_amdgcn_ldexpf(act_plain<ACT>(acc[mb][4 * i + jj]), -sg);
                                h[i][0] = pack_f16x2(v[0], v[1]);
                                h[i][1] = pack_f16x2(v[2], v[3]);
                            }
                            store_glu(g, h);
                            if (half == 0) {
                                prm.gexp[(long long)(2 * fc) * prm.p_cap + r] = (int8_t)sg;
                                prm.gexp[(long long)(2 * fc + 1) * prm.p_cap + r] = (int8_t)sg;
                            }
                            mark_scaled(r);
                        }
                    }
                }
            } else {
                // Y rows as 24-bit floats (fp32 rounded to 16 mantissa bits, 2^-16 relative): the combine sums
                // the K rows of a token from nearly exact values, at 3/4 of fp32's bytes. A lane packs its four
                // groups of four columns (8i + c4 + jj) into 12 bytes each; exchanging groups 0, 1 of lane
                // l + 32 for groups 2, 3 of lane l (three dwords each) leaves lane l columns 0-15 of the row
                // and lane l + 32 columns 16-31, 48 contiguous bytes each: three 16-byte stores (aligned: H is
                // a multiple of 64) instead of four 12-byte ones.
                unsigned char* Yb = reinterpret_cast<unsigned char*>(prm.out);
                const float wsc = __builtin_amdgcn_ldexpf(1.0f, s_wx[tb][wave]);  // the fragment's fp16 scale
#pragma unroll
                for (int mb = 0; mb < kPkMB; ++mb) {
                    if (mb >= nmb) break;
                    const int row = mb * 32 + lrow;
                    if (row < rows) {  // lanes l and l ^ 32 hold the same row, so both run this or neither
                        const float ws = wsc * s_w[tb][row];  // exact: wsc is a power of two
                        const long long p = s_pair[tb][row];
                        f24x4 q[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            q[i] = pack_f24x4(acc[mb][4 * i] * ws, acc[mb][4 * i + 1] * ws, acc[mb][4 * i + 2] * ws,
                                              acc[mb][4 * i + 3] * ws);
#pragma unroll
                        for (int d = 0; d < 3; ++d) {
                            swap_halves(q[0].d[d], q[2].d[d]);
                            swap_halves(q[1].d[d], q[3].d[d]);
                        }
                        u32x4* yrow = reinterpret_cast<u32x4*>(Yb + (p * prm.H + 32 * fc + 16 * half) * 3);
                        yrow[0] = u32x4{q[0].d[0], q[0].d[1], q[0].d[2], q[2].d[0]};
                        yrow[1] = u32x4{q[2].d[1], q[2].d[2], q[1].d[0], q[1].d[1]};
                        yrow[2] = u32x4{q[1].d[2], q[3].d[0], q[3].d[1], q[3].d[2]};
                    }
                }
            }
        }
        lds_barrier();  // s_next
        // The same value in every lane; readfirstlane tells the compiler so, which keeps the item decode and
        // the operand descriptors in scalar registers (otherwise every weight load gets a waterfall loop).
        const int it_nn = __builtin_amdgcn_readfirstlane(s_next);
        if (!has_nx) {  // tickets are drawn in increasing order: the held one is past the end too
            // the prefetch copies into LDS land before the workgroup (and its LDS) is gone
            __builtin_amdgcn_s_waitcnt(0x0F70);
            return false;
        }
        it_nx = it_nn;
        if (tid == 0) ticket = atomicAdd(prm.counters + xcd, 1);
        cur = nx;
        ra_cur = ra_nx;
        rb_cur = rb_nx;
        bstep_cur = bstep_nx;
        if constexpr (!XPF) start_item(cur, tb ^ 1);
        return true;
    };
    for (int j = 0;; ++j)
        if (!item(j)) break;
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

// Workgroups of a packed GEMM launch: one per CU, a multiple of 8 (the same count on every XCD).
static int pk_grid(int max_tiles, int n_tiles) {
    const int grid = (int)std::min<long long>((long long)max_tiles * n_tiles, pk_cu_count());
    return ceil_div(max(grid, 1), 8) * 8;
}

template <int MODE, int ACT, bool HAS_BIAS>
static hipError_t launch_pk_t(const PkParams& prm, int max_tiles, hipStream_t s) {
    const int grid = pk_grid(max_tiles, prm.n_tiles);
    const int nst = prm.Kd / kBK;
    if (nst < 2)
        hipLaunchKernelGGL((moe_gemm_packed_kernel<MODE, ACT, HAS_BIAS, false, 1, false>), dim3(grid), dim3(kPkThreads), 0, s, prm);
    else if (nst % 3 == 0)
        hipLaunchKernelGGL((moe_gemm_packed_kernel<MODE, ACT, HAS_BIAS, true, 0, false>), dim3(grid), dim3(kPkThreads), 0, s, prm);
    else if (nst % 3 == 1)
        hipLaunchKernelGGL((moe_gemm_packed_kernel<MODE, ACT, HAS_BIAS, true, 1, false>), dim3(grid), dim3(kPkThreads), 0, s, prm);
    else if (nst >= 5)
        hipLaunchKernelGGL((moe_gemm_packed_kernel<MODE, ACT, HAS_BIAS, true, 2, true>), dim3(grid), dim3(kPkThreads), 0, s, prm);
    else
        hipLaunchKernelGGL((moe_gemm_packed_kernel<MODE, ACT, HAS_BIAS, true, 2, false>), dim3(grid), dim3(kPkThreads), 0, s, prm);
    return hipGetLastError();
}

hipError_t launch_route(const int32_t* idx, int T, int K, int E, int BM, int32_t* offsets, int32_t* sorted_pairs,
                        int32_t* tile_offsets, int32_t* tile_expert, int32_t* meta, int32_t* counts,
                        int32_t* sched, hipStream_t stream, int8_t* row_zero = nullptr,
                        const XcdSplit* split = nullptr);
// out[t, :] = bf16( sum over valid slots k of Y[t*K + k, :] * 2^psig + w[t, k] * b2[e] ), slots in k
// order, Y in the 24-bit float form both down GEMMs write (the packed one: w * glu W2, without the bias;
// psig only when some glu row was stored scaled, i.e. sync non-null and sync[1] set; the stored-layout one:
// w * (glu W2 + b2), with bias and sync null). One workgroup per token, H/8 threads rounded up to whole
// waves; a thread owns 8 consecutive columns (two 12-byte loads per slot) and issues the loads of four
// slots before it adds them, still in slot order.
__global__ __launch_bounds__(1024) void moe_combine_h_kernel(const unsigned char* __restrict__ Yb,
                                                            const int32_t* __restrict__ idx, uint16_t* __restrict__ out,
                                                            int T, int K, int E, int H,
                                                            const int32_t* __restrict__ sync,
                                                            const int8_t* __restrict__ psig,
                                                            const float* __restrict__ bias, const float* __restrict__ route_w) {
    const int t = blockIdx.x;
    const bool scaled = sync != nullptr && sync[1] != 0;  // some glu row was stored scaled: its Y row is scaled by 2^-psig
    for (int c = threadIdx.x; c < H / 8; c += blockDim.x) {
        f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
        for (int k0 = 0; k0 < K; k0 += 4) {
            f24x4 q[4][2];
            int ev[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int k = k0 + j;
                ev[j] = k < K ? idx[t * K + k] : -1;
                if ((unsigned)ev[j] < (unsigned)E) {
                    const unsigned char* src = Yb + (((long long)t * K + k) * H + 8 * c) * 3;
                    __builtin_memcpy(&q[j][0], src, 12);
                    __builtin_memcpy(&q[j][1], src + 12, 12);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int k = k0 + j, e = ev[j];
                if ((unsigned)e >= (unsigned)E) continue;
                f32x4 y0 = unpack_f24x4(q[j][0]), y1 = unpack_f24x4(q[j][1]);
                if (scaled) {
                    const float sc = __builtin_amdgcn_ldexpf(1.0f, psig[(long long)t * K + k]);
                    y0 *= sc;
                    y1 *= sc;
                }
                if (bias) {  // the slot's share of the down bias, w * b[e]
                    const float w = route_w[(long long)t * K + k];
                    const f32x4* bb = reinterpret_cast<const f32x4*>(bias + (long long)e * H + 8 * c);
                    y0 += w * bb[0];
                    y1 += w * bb[1];
                }
                s0 += y0;
                s1 += y1;
            }
        }
        *reinterpret_cast<u32x4*>(out + (long long)t * H + 8 * c) =
            u32x4{pack_bf16x2(s0[0], s0[1]), pack_bf16x2(s0[2], s0[3]), pack_bf16x2(s1[0], s1[1]), pack_bf16x2(s1[2], s1[3])};
    }
}

// Between the GEMMs: glu rows with a segment stored scaled (rsig[r] != 0, marked by GEMM1) are brought
// to the largest scale s_r of the row's segments (all-zero segments, kGluAnyScale, take any scale and
// are left alone; the others are rescaled by 2^-(s_r - s_u), fp16 round to nearest), and psig[pair] =
// s_r for every valid pair (the combine multiplies the pair's Y row by 2^s_r; the down bias is added
// there unscaled). rsig[r] is only the mark; it is set to s_r for inspection and read by no kernel.
// Exits at once unless GEMM1 marked some row (sync[1]).
__global__ __launch_bounds__(256) void moe_glu_fixup_kernel(uint16_t* __restrict__ glu, const int8_t* __restrict__ gexp,
                                                            int8_t* __restrict__ rsig, int8_t* __restrict__ psig,
                                                            const int32_t* __restrict__ sorted_pairs,
                                                            const int32_t* __restrict__ sync,
                                                            const int32_t* __restrict__ meta, int p_cap, int F) {
    if (sync[1] == 0) return;
    const int nrows = meta[1], U16 = F / 16;
    for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < nrows; r += gridDim.x * blockDim.x) {
        if (rsig[r] == 0) {
            psig[sorted_pairs[r]] = 0;
            continue;
        }
        int smax = kGluAnyScale;  // a marked row has a scaled segment, so smax ends above kGluAnyScale
        for (int u = 0; u < U16; ++u) smax = max(smax, (int)gexp[(long long)u * p_cap + r]);
        for (int u = 0; u < U16; ++u) {
            const int su = gexp[(long long)u * p_cap + r];
            const int d = smax - su;
            if (d == 0 || su == kGluAnyScale) continue;
            uint16_t* g = glu + (long long)r * F + 16 * u;
            for (int j = 0; j < 16; ++j) {
                const float v = (float)__builtin_bit_cast(_Float16, g[j]);
                g[j] = __builtin_bit_cast(uint16_t, (_Float16)__builtin_amdgcn_ldexpf(v, -d));
            }
        }
        rsig[r] = (int8_t)smax;
        psig[sorted_pairs[r]] = (int8_t)smax;
    }
}

int packed_tile_m() { return kPkBM; }

// Fragments per item. Items of one projection all have the same cost, so a launch takes
// ceil(items / CUs) rounds; narrower items (fewer active waves) cut the last, partly empty round at
// the price of more items. Estimated from the shape alone (rows per expert P/E, no device sync): an
// item stage costs max(weight streaming ~ fw, MFMA of the busiest SIMD ~ ceil(fw/4) * blocks), plus
// a fixed epilogue per item. Prefers wider items unless a narrower one is 2% cheaper.
static int pick_fw(long long P, int E, int NF, int Kd, int cus) {
    const double r = (double)P / E;
    const int mt_e = std::max(1, (int)std::ceil(r / kPkBM));                       // M-tiles per expert
    const int nmb = std::max(1, (int)std::ceil(std::min<double>(kPkBM, r) / 32));  // blocks per M-tile
    const long long mtiles = (long long)E * mt_e;
    const int nst = Kd / kBK;
    double best = 0;
    int best_w = kPkWaves;
    for (int w = kPkWaves; w >= 1; --w) {
        const long long items = mtiles * ceil_div(NF, w);
        const long long rounds = (items + cus - 1) / cus;
        const double stage = std::max(w * 175.0 / mt_e, ceil_div(w, 4) * nmb * 64.0);
        const double cost = rounds * (nst * stage + 2000.0);
        if (w == kPkWaves || cost < best * 0.98) {
            best = cost;
            best_w = w;
        }
    }
    return best_w;
}

hipError_t launch_combine_h(const unsigned char* Y, const int32_t* idx, uint16_t* out, int T, int K, int E, int H,
                            const int32_t* sync, const int8_t* psig, const float* b2, const float* route_w,
                            hipStream_t s);

// route -> packed gate_up GEMM -> packed down GEMM -> combine, all on stream s. Shapes were checked
// by the caller (H % 64 == 0, F % 64 == 0, E <= 1024, T >= 1).
hipError_t launch_prefill_packed(const void* x, const void* w1p, const float* b1, const void* w2p, const float* b2,
                                 const int32_t* idx, const float* route_w, int T, int H, int F, int E, int K,
                                 int bias_interleaved, int act, void* out, int32_t* offsets, int32_t* tile_offsets,
                                 int32_t* meta, int32_t* sorted_pairs, int32_t* tile_expert, int32_t* route_counts,
                                 int max_tiles, uint16_t* glu, float* Y, int8_t* gexp, int8_t* rsig,
                                 int8_t* psig, hipStream_t s, hipEvent_t* ev) {
    auto mark = [&](int i) { if (ev) (void)hipEventRecord(ev[i], s); };
    // Launch shapes of both GEMMs, from the shape alone; the route then splits each one's items over
    // the XCDs (meta[32..40] gate_up, meta[41..49] down). Where even the most M-tiles the route can
    // make (ceil(P / 256) + min(P, E)) would give each workgroup fewer than 8 rounds of items, the
    // split is the equal one for both GEMMs (moe_split.h) and the GEMMs compute it themselves.
    const int nf1 = act_is_gated(act) ? F / 16 : F / 32, nf2 = H / 32;
    const int fw1 = pick_fw((long long)T * K, E, nf1, H, pk_cu_count());
    const int fw2 = pick_fw((long long)T * K, E, nf2, F, pk_cu_count());
    const int nt1 = ceil_div(nf1, fw1), nt2 = ceil_div(nf2, fw2);
    const int slots1 = pk_grid(max_tiles, nt1) / 8, slots2 = pk_grid(max_tiles, nt2) / 8;
    const long long P = (long long)T * K, mt_max = (P + kPkBM - 1) / kPkBM + std::min<long long>(P, E);
    auto max_rounds = [&](int nt, int slots) { return (mt_max * nt + 8LL * slots - 1) / (8LL * slots); };
    const bool cost_split = max(max_rounds(nt1, slots1), max_rounds(nt2, slots2)) >= 8;
    XcdSplit split{{fw1, fw2}, {nt1, nt2}, {slots1, slots2}, meta + 32};
    mark(0);
    hipError_t st =
        launch_route(idx, T, K, E, kPkBM, offsets, sorted_pairs, tile_offsets, tile_expert, meta, route_counts,
                     meta + 8, s, rsig, cost_split ? &split : nullptr);
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
    g1.bounds = cost_split ? meta + 32 : nullptr;
    g1.route_w = route_w;
    g1.out = glu;
    g1.Kd = H;
    g1.NF = nf1;
    g1.KS = H / 16;
    g1.fw = fw1;
    g1.n_tiles = nt1;
    g1.F = F;
    g1.H = H;
    g1.topk = K;
    g1.bias_interleaved = bias_interleaved;
    g1.a_bytes = T * H * 2;
    g1.counters = meta + 8;
    g1.gexp = gexp;
    g1.rsig = rsig;
    g1.sync = meta + 24;
    g1.p_cap = T * K;
    g1.tail = (long long)T * K < (long long)kPkBM * E ? kPkTailGateUp : 0;  // fewer rows per expert than one M-tile
    if (act == kActSilu)
        st = b1 ? launch_pk_t<kModePkGateUp, kActSilu, true>(g1, max_tiles, s)
                : launch_pk_t<kModePkGateUp, kActSilu, false>(g1, max_tiles, s);
    else if (act == kActGptOss)
        st = b1 ? launch_pk_t<kModePkGateUp, kActGptOss, true>(g1, max_tiles, s)
                : launch_pk_t<kModePkGateUp, kActGptOss, false>(g1, max_tiles, s);
    else if (act == kActGeluTanh)  // non-gated: no first-projection bias (checked by the caller)
        st = launch_pk_t<kModePkUp, kActGeluTanh, false>(g1, max_tiles, s);
    else if (act == kActSiluPlain)
        st = launch_pk_t<kModePkUp, kActSiluPlain, false>(g1, max_tiles, s);
    else
        st = launch_pk_t<kModePkUp, kActRelu, false>(g1, max_tiles, s);
    if (st != hipSuccess) return st;
    hipLaunchKernelGGL(moe_glu_fixup_kernel, dim3(32), dim3(256), 0, s, glu, gexp, rsig, psig, sorted_pairs, meta + 24,
                       meta, T * K, F);
    st = hipGetLastError();
    if (st != hipSuccess) return st;
    mark(2);
    PkParams g2 = g1;
    g2.A = glu;
    g2.B = static_cast<const uint16_t*>(w2p);
    g2.out = Y;  // written as 24-bit floats (3/4 of the fp32 buffer)
    g2.wexp = reinterpret_cast<const int8_t*>(static_cast<const uint16_t*>(w2p) + (long long)E * H * F);
    g2.Kd = F;
    g2.NF = nf2;
    g2.KS = F / 16;
    g2.fw = fw2;
    g2.counters = meta + 16;
    g2.n_tiles = nt2;
    g2.bounds = cost_split ? meta + 41 : nullptr;
    g2.bias = nullptr;  // the down bias is added by the combine
    g2.tail = 0;
    st = launch_pk_t<kModePkDown, kActSilu, false>(g2, max_tiles, s);
    if (st != hipSuccess) return st;
    mark(3);
    st = launch_combine_h(reinterpret_cast<const unsigned char*>(Y), idx, static_cast<uint16_t*>(out), T, K, E, H,
                          meta + 24, psig, b2, route_w, s);
    mark(4);
    return st;
}

hipError_t launch_combine_h(const unsigned char* Y, const int32_t* idx, uint16_t* out, int T, int K, int E, int H,
                            const int32_t* sync, const int8_t* psig, const float* b2, const float* route_w,
                            hipStream_t s) {
    if (T == 0) return hipSuccess;
    hipLaunchKernelGGL(moe_combine_h_kernel, dim3(T), dim3(std::min(1024, ceil_div(H / 8, kWave) * kWave)), 0, s, Y,
                       idx, out, T, K, E, H, sync, psig, b2, route_w);
    return hipGetLastError();
}

}  // namespace cmoe
