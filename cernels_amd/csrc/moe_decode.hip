// Decode path (few tokens): fused gather-GEMV over the selected experts only.
//
// Replaces decode_gateup_swiglu_kernel / decode_down_accum_kernel + zeros + cast
// (src/kops/cohere2_moe_experts/csrc/cohere2_moe_experts.cu:135-236). Differences by design:
//   * the gate_up GEMV is split by DISTINCT expert, so an expert picked by several
//     (token, slot) pairs streams its gate_up rows from HBM once (the reference streams them once
//     per pair, .cu:143);
//   * 64-lane waves read whole 1 KB runs of a weight row per instruction (16 bytes per lane) and
//     keep every row they own in flight at once; dot products use v_dot2c_f32_bf16;
//   * the top-k combine is fused into the down GEMV: a workgroup owns whole output rows and sums
//     every (token, slot) contribution for them in a fixed order, then writes bf16 — no fp32
//     atomics, no cross-workgroup synchronisation, no zero-fill or cast kernel. Two launches.
//
// Layout: concat only (gate_up [E, 2F, H], down [E, H, F]); the reference has no decode entry
// for the interleaved gpt-oss layout either.
#include <mutex>

#include "moe_common.h"
#include "../../include/cernels_moe.h"

namespace cmoe {

constexpr int kDecThreads = 256;
constexpr int kDecWaves = kDecThreads / kWave;
constexpr int kDecMaxPairs = 256;
constexpr int kDecMaxTokens = 64;
constexpr int kDecMaxExperts = 1024;  // bitmap of 32 words
constexpr int kDnWaves = 8;           // waves per down workgroup
constexpr int kDnThreads = kDnWaves * kWave;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// 8-element bf16 dot product, fp32 accumulate. The vectors are reinterpreted whole and split with
// shufflevector: a bit_cast of a single vector-element lvalue (a[d]) reads element 0 whatever d is.
__device__ __forceinline__ float dot8(const u32x4& a, const u32x4& b, float acc) {
    const bf16x8 av = __builtin_bit_cast(bf16x8, a), bv = __builtin_bit_cast(bf16x8, b);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(av, av, 0, 1), __builtin_shufflevector(bv, bv, 0, 1),
                                          acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(av, av, 2, 3), __builtin_shufflevector(bv, bv, 2, 3),
                                          acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(av, av, 4, 5), __builtin_shufflevector(bv, bv, 4, 5),
                                          acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(av, av, 6, 7), __builtin_shufflevector(bv, bv, 6, 7),
                                          acc, false);
    return acc;
}

// Lane-strided row chunks: lane l holds 16-byte chunks l, l+64, ... of a row of nch chunks.
template <int MAXC>
__device__ __forceinline__ void load_row(const uint16_t* __restrict__ row, int nch, int lane, u32x4 (&v)[MAXC]) {
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
        const int c = lane + kWave * i;
        if (c < nch) v[i] = *reinterpret_cast<const u32x4*>(row + 8 * c);
        else v[i] = u32x4{0u, 0u, 0u, 0u};
    }
}

// Value of lane l ^ o for o = 1, 2, 8 through DPP (quad_perm, row_ror:8: exact xor partners within a row of 16
// lanes), else through ds_bpermute.
template <int O>
__device__ __forceinline__ float xor_lane(float v) {
    const int b = __builtin_bit_cast(int, v);
    if constexpr (O == 1) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(b, 0xB1, 0xF, 0xF, false));
    else if constexpr (O == 2) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(b, 0x4E, 0xF, 0xF, false));
    else if constexpr (O == 8) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(b, 0x128, 0xF, 0xF, false));
    else return __shfl_xor(v, O, kWave);
}

// Sum of N per-lane values over the wave, several values per exchange: after the halving steps
// (offsets 32, 16, ... while more than G values remain), each lane holds G values that are sums over
// the lanes sharing its upper bits; the remaining single-offset steps complete those G sums in every
// lane. On return, v[0..G) of lane l hold totals of the value group selected by l's upper bits:
// group index = lane >> (6 - log2(N/G)). The completing steps need not pair lane l with l ^ o, only
// cover the group: offset 4 uses row_half_mirror (l <-> 7 - l within eight lanes), which with the
// xor-1 and xor-2 steps after it still sums all eight lanes. Lanes of a group may round their totals
// differently; callers read one fixed lane per group.
template <int N, int G, int O>
__device__ __forceinline__ void reduce_step_halving(float (&v)[N], int lane, int n) {
    const bool upper = lane & O;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
        if (i >= n / 2) break;
        const float send = upper ? v[i] : v[i + n / 2];
        const float keep = upper ? v[i + n / 2] : v[i];
        v[i] = keep + xor_lane<O>(send);
    }
}
template <int G, int O>
__device__ __forceinline__ float complete_step(float x) {
    if constexpr (O == 4)
        return x + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x141, 0xF, 0xF, false));
    else return x + xor_lane<O>(x);
}
template <int N, int G>
__device__ __forceinline__ void wave_reduce_groups(float (&v)[N], int lane) {
    static_assert(N >= G && G >= 1 && (N & (N - 1)) == 0 && (G & (G - 1)) == 0, "powers of two");
    constexpr int H = N / G;  // halving steps: log2(H), offsets 32, 16, ...
    static_assert(H <= 8, "halving steps use offsets 32, 16, 8");
    if constexpr (H >= 2) reduce_step_halving<N, G, 32>(v, lane, N);
    if constexpr (H >= 4) reduce_step_halving<N, G, 16>(v, lane, N / 2);
    if constexpr (H >= 8) reduce_step_halving<N, G, 8>(v, lane, N / 4);
#pragma unroll
    for (int i = 0; i < G; ++i) {
        float x = v[i];
        if constexpr (H < 2) x = complete_step<G, 32>(x);
        if constexpr (H < 4) x = complete_step<G, 16>(x);
        if constexpr (H < 8) x = complete_step<G, 8>(x);
        x = complete_step<G, 4>(x);
        x = complete_step<G, 2>(x);
        x = complete_step<G, 1>(x);
        v[i] = x;
    }
}

// glu[p, f] = bf16(act(x[t_p] . W1_e[f] + b1_e[f], x[t_p] . W1_e[F+f] + b1_e[F+f])) for the pairs p
// of one distinct expert e.
// grid: (ceil(F / (4 * R)), min(T*K, E)); blockIdx.y = u picks the u-th smallest distinct expert
// (waves past the number of distinct experts return at once). Wave w owns R consecutive f and
// keeps their 2R weight rows in registers for all of e's pairs. Every wave finds e and its pairs
// on its own (its own LDS bitmap and pair list, ballots, no workgroup barrier), loads the first
// pair's x row ahead of its weight rows and each further pair's x row while the previous pair is
// reduced. Measured against one workgroup-wide selection (two barriers, x row loaded per pair):
// 29.9 -> 28.9 us at T=8 (H=1280) and 10.6 -> 10.3 us at T=1 (H=2048).
template <int ACT, bool HAS_BIAS, int MAXC, int R>
__global__ __launch_bounds__(kDecThreads) void moe_decode_gateup_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1, const float* __restrict__ b1,
    const int32_t* __restrict__ idx, uint16_t* __restrict__ glu, int32_t* __restrict__ order, int T, int H, int F,
    int E, int K) {
    __shared__ uint32_t bits[kDecWaves][kDecMaxExperts / 32];
    __shared__ int plist[kDecWaves][kDecMaxPairs];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int P = T * K, u = blockIdx.y;
    const int f0 = (blockIdx.x * kDecWaves + wave) * R;
    if (f0 >= F) return;  // wave-uniform; nothing below synchronises the workgroup

    // ---- the pairs' expert ids, four 64-pair chunks (P <= 256 is checked on the host)
    int ev[kDecMaxPairs / kWave];
#pragma unroll
    for (int c = 0; c < kDecMaxPairs / kWave; ++c) {
        const int p = lane + kWave * c;
        const int v = p < P ? idx[p] : -1;
        ev[c] = ((unsigned)v < (unsigned)E) ? v : -1;
    }
    // Wave 0 of the first row group of each expert publishes that expert's pairs in the pair order the down
    // GEMV walks (by expert, then by pair); the one of expert 0 also marks the entries past the valid pairs.
    const bool lead = blockIdx.x == 0 && wave == 0;
    if (lead && u == 0) {
        int nv = 0;
#pragma unroll
        for (int c = 0; c < kDecMaxPairs / kWave; ++c) nv += __popcll(__ballot(ev[c] >= 0));
#pragma unroll
        for (int c = 0; c < kDecMaxPairs / kWave; ++c)
            if (nv + lane + kWave * c < P) order[nv + lane + kWave * c] = -1;
    }
    // ---- this wave's bitmap of valid expert ids (its own LDS words; LDS ops of a wave run in order)
    uint32_t* wb = bits[wave];
    if (lane < kDecMaxExperts / 32) wb[lane] = 0u;
#pragma unroll
    for (int c = 0; c < kDecMaxPairs / kWave; ++c)
        if (ev[c] >= 0) atomicOr(&wb[ev[c] >> 5], 1u << (ev[c] & 31));
    uint32_t bw = lane < kDecMaxExperts / 32 ? wb[lane] : 0u;
    const int cnt = __popc(bw);  // 0..32
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
    // exclusive prefix sum of cnt over the lower lanes, bit by bit of cnt (ballots, no LDS round trips)
    int excl = 0;
#pragma unroll
    for (int b = 0; b < 6; ++b) excl += __popcll(__ballot((cnt >> b) & 1) & lt) << b;
    const int incl = excl + cnt;
    const bool holder = u >= excl && u < incl;  // at most one lane
    int eh = 0;
    if (holder) {
        for (int r = u - excl; r > 0; --r) bw &= bw - 1;
        eh = lane * 32 + __ffs(bw) - 1;
    }
    const uint64_t hb = __ballot(holder);
    if (hb == 0ull) return;  // fewer distinct experts than u + 1
    const int e = __builtin_amdgcn_readlane(eh, __ffsll((unsigned long long)hb) - 1);

    // ---- pairs of e, ascending p, into this wave's list
    int np = 0, base = 0;  // base: valid pairs of smaller expert ids (lead wave only)
    if (lead) {
#pragma unroll
        for (int c = 0; c < kDecMaxPairs / kWave; ++c) base += __popcll(__ballot(ev[c] >= 0 && ev[c] < e));
    }
#pragma unroll
    for (int c = 0; c < kDecMaxPairs / kWave; ++c) {
        const bool mine = ev[c] == e;
        const uint64_t mk = __ballot(mine);
        if (mine) {
            const int at = np + __popcll(mk & lt);
            plist[wave][at] = kWave * c + lane;
            if (lead) order[base + at] = (e << 16) | (kWave * c + lane);
        }
        np += __popcll(mk);
    }
    int ip = 0;
    auto pop = [&]() -> int { return ip < np ? __builtin_amdgcn_readfirstlane(plist[wave][ip++]) : -1; };
    const int nch = H / 8;
    int p = pop();
    u32x4 xs[2][MAXC];
    load_row<MAXC>(x + (long long)(p / K) * H, nch, lane, xs[0]);

    // ---- this wave's 2R weight rows
    const uint16_t* we = w1 + (long long)e * 2 * F * H;
    u32x4 wr[2 * R][MAXC];  // rows: gate f0, up f0, gate f0+1, up f0+1, ...
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int f = min(f0 + r, F - 1);
        load_row<MAXC>(we + (long long)f * H, nch, lane, wr[2 * r]);
        load_row<MAXC>(we + (long long)(F + f) * H, nch, lane, wr[2 * r + 1]);
    }
    int pn = pop();
    if (pn >= 0) load_row<MAXC>(x + (long long)(pn / K) * H, nch, lane, xs[1]);

    constexpr int gr_shift = 6 - (R == 1 ? 0 : (R == 2 ? 1 : (R == 4 ? 2 : 3)));
    const int my_r = lane >> gr_shift;
    float bg = 0.f, bu = 0.f;
    if constexpr (HAS_BIAS) {
        const int f = min(f0 + my_r, F - 1);
        bg = b1[(long long)e * 2 * F + f];
        bu = b1[(long long)e * 2 * F + F + f];
    }
    const bool writer = (lane & ((1 << gr_shift) - 1)) == 0 && f0 + my_r < F;
    auto emit = [&](int pp, auto bc) {
        constexpr int B = decltype(bc)::value;
        float v[2 * R];
#pragma unroll
        for (int j = 0; j < 2 * R; ++j) {
            v[j] = 0.f;
#pragma unroll
            for (int i = 0; i < MAXC; ++i) v[j] = dot8(wr[j][i], xs[B][i], v[j]);
        }
        wave_reduce_groups<2 * R, 2>(v, lane);
        if (writer) glu[(long long)pp * F + f0 + my_r] = f32_to_bf16_bits(swiglu<ACT>(v[0] + bg, v[1] + bu));
    };
    for (;;) {
        emit(p, std::integral_constant<int, 0>{});
        if (pn < 0) break;
        p = pn;
        pn = pop();
        if (pn >= 0) load_row<MAXC>(x + (long long)(pn / K) * H, nch, lane, xs[0]);
        emit(p, std::integral_constant<int, 1>{});
        if (pn < 0) break;
        p = pn;
        pn = pop();
        if (pn >= 0) load_row<MAXC>(x + (long long)(pn / K) * H, nch, lane, xs[1]);
    }
}

// out[t, h] = bf16( sum over valid slots k of w_{t,k} * (glu[t*K+k] . W2_{e}[h] + b2_e[h]) ).
// grid: ceil(H / HB), 8 waves; HB = 4 output rows per workgroup while that still leaves two workgroups per CU
// and rows are short (F <= 1024), else 2. The valid pairs, sorted by expert and then by pair (order[P], written by
// the gate_up launch; -1 past the valid pairs), are cut into eight consecutive runs, one per wave. A wave walks
// its run QB pairs at a time (all their down rows and glu rows in flight together) and loads an expert's rows
// only where the expert changes: consecutive pairs of one expert reuse the rows already in registers. Each lane
// accumulates the sums of the token it holds; the eight waves' partial sums are added in wave order at the end,
// so the result does not depend on timing. Run entries are wave-uniform (scalar loads).
template <bool HAS_BIAS, int MAXC, int QB, int HB>
__global__ __launch_bounds__(kDnThreads) void moe_decode_down_kernel(
    const uint16_t* __restrict__ glu, const uint16_t* __restrict__ w2, const float* __restrict__ b2,
    const int32_t* __restrict__ order, const float* __restrict__ route_w, uint16_t* __restrict__ out, int T, int H,
    int F, int K) {
    static_assert(QB == 1 || QB == 2, "pairs per batch");
    __shared__ float part[kDnWaves][HB][kDecMaxTokens];
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int h0 = blockIdx.x * HB;
    const int nch = F / 8, P = T * K;
    const int run = ceil_div(P, kDnWaves);
    const int i0 = wave * run, i1 = min(i0 + run, P);
    float acc[HB];
#pragma unroll
    for (int j = 0; j < HB; ++j) acc[j] = 0.f;  // lane t holds token t's sums

    u32x4 wr[QB][HB][MAXC], gv[QB][MAXC];
    auto rows = [&](int e, auto sc) {
        constexpr int S = decltype(sc)::value;
        const uint16_t* we = w2 + (long long)e * H * F;
#pragma unroll
        for (int j = 0; j < HB; ++j) load_row<MAXC>(we + (long long)min(h0 + j, H - 1) * F, nch, lane, wr[S][j]);
    };
    int prev_e = -1, prev_slot = 0;  // expert whose rows the registers hold, and in which slot
    for (int i = i0; i < i1; i += QB) {
        const int o0 = order[i];
        if (o0 < 0) break;  // past the valid pairs (wave-uniform)
        const int o1r = QB == 2 && i + 1 < i1 ? order[i + 1] : -1;
        const bool two = o1r >= 0;  // wave-uniform
        const int o1 = two ? o1r : o0;
        const int e0 = o0 >> 16, p0 = o0 & 0xffff, e1 = o1 >> 16, p1 = o1 & 0xffff;
        if (e0 != prev_e) rows(e0, std::integral_constant<int, 0>{});
        else if constexpr (QB == 2) {
            if (prev_slot == 1) {
#pragma unroll
                for (int j = 0; j < HB; ++j)
#pragma unroll
                    for (int c = 0; c < MAXC; ++c) wr[0][j][c] = wr[QB - 1][j][c];
            }
        }
        const bool same = e1 == e0;
        if constexpr (QB == 2) {
            if (!same) rows(e1, std::integral_constant<int, QB - 1>{});
        }
        load_row<MAXC>(glu + (long long)p0 * F, nch, lane, gv[0]);
        if constexpr (QB == 2) {
            load_row<MAXC>(glu + (long long)p1 * F, nch, lane, gv[QB - 1]);
            if (same) {  // after the glu loads are issued: the copy waits for the rows only
#pragma unroll
                for (int j = 0; j < HB; ++j)
#pragma unroll
                    for (int c = 0; c < MAXC; ++c) wr[QB - 1][j][c] = wr[0][j][c];
            }
        }
        float d[QB * HB];
#pragma unroll
        for (int q = 0; q < QB; ++q)
#pragma unroll
            for (int j = 0; j < HB; ++j) {
                d[q * HB + j] = 0.f;
#pragma unroll
                for (int c = 0; c < MAXC; ++c) d[q * HB + j] = dot8(wr[q][j][c], gv[q][c], d[q * HB + j]);
            }
        wave_reduce_groups<QB * HB, 1>(d, lane);  // value v's total sits in lanes [v*64/(QB*HB), ...)
#pragma unroll
        for (int q = 0; q < QB; ++q) {
            if (q == 1 && !two) break;  // wave-uniform
            const int pp = q == 0 ? p0 : p1, ee = q == 0 ? e0 : e1;
            const float wp = route_w[pp];
            const int t = pp / K;
#pragma unroll
            for (int j = 0; j < HB; ++j) {
                const float dj = __builtin_bit_cast(
                    float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, d[0]), (q * HB + j) * (kWave / (QB * HB))));
                float bj = 0.f;
                if constexpr (HAS_BIAS) bj = b2[(long long)ee * H + min(h0 + j, H - 1)];
                if (lane == t) acc[j] += wp * (dj + bj);
            }
        }
        prev_e = two ? e1 : e0;
        prev_slot = two ? 1 : 0;
    }
#pragma unroll
    for (int j = 0; j < HB; ++j) part[wave][j][lane] = acc[j];
    __syncthreads();
    for (int i = tid; i < HB * T; i += kDnThreads) {
        const int j = i / T, t = i - j * T, h = h0 + j;
        if (h >= H) continue;
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < kDnWaves; ++w) sum += part[w][j][t];
        out[(long long)t * H + h] = f32_to_bf16_bits(sum);
    }
}

int decode_max_pairs() { return kDecMaxPairs; }
int decode_max_tokens() { return kDecMaxTokens; }

template <int ACT, bool HAS_BIAS, int MAXC, int R>
static void launch_gateup_r(const uint16_t* x, const uint16_t* w1, const float* b1, const int32_t* idx, uint16_t* glu,
                            int32_t* order, int T, int H, int F, int E, int K, hipStream_t s) {
    dim3 grid(ceil_div(F, kDecWaves * R), min(T * K, E));
    hipLaunchKernelGGL((moe_decode_gateup_kernel<ACT, HAS_BIAS, MAXC, R>), grid, dim3(kDecThreads), 0, s, x, w1, b1,
                       idx, glu, order, T, H, F, E, K);
}

static int g_dec_cu_count = 0;

static int dec_cu_count() {
    if (g_dec_cu_count == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            g_dec_cu_count = n;
        else
            g_dec_cu_count = 256;
    }
    return g_dec_cu_count;
}

// R (f per wave) = 2: four weight rows in flight per wave. Measured against R = 1 and R = 4 on both decode
// workloads: R = 4 (eight rows, fewer and larger workgroups) was 2.5 us slower at T=8, H=1280 and
// 1.4 us slower at T=1, H=2048; R = 1 was within noise of R = 2.
template <int ACT, bool HAS_BIAS, int MAXC>
static void launch_gateup_t(const uint16_t* x, const uint16_t* w1, const float* b1, const int32_t* idx, uint16_t* glu,
                            int32_t* order, int T, int H, int F, int E, int K, hipStream_t s) {
    launch_gateup_r<ACT, HAS_BIAS, MAXC, 2>(x, w1, b1, idx, glu, order, T, H, F, E, K, s);
}

// QB (pairs per batch) is 2 while rows are short (F <= 2048) and a wave has more than one pair, else 1, to bound
// the registers they take. Four output rows per workgroup when H / 4 still fills every CU twice: fewer, larger
// workgroups stream the same rows with less per-workgroup overhead. With two rows, two pairs per batch keep
// three workgroups per CU resident, so T=8's 640 workgroups (H=1280) run in one wave of residency.
template <bool HAS_BIAS, int MAXC, int QB, int HB>
static void launch_down_k(const uint16_t* glu, const uint16_t* w2, const float* b2, const int32_t* order,
                          const float* route_w, uint16_t* out, int T, int H, int F, int K, hipStream_t s) {
    hipLaunchKernelGGL((moe_decode_down_kernel<HAS_BIAS, MAXC, QB, HB>), dim3(ceil_div(H, HB)), dim3(kDnThreads), 0, s,
                       glu, w2, b2, order, route_w, out, T, H, F, K);
}
template <bool HAS_BIAS, int MAXC>
static void launch_down_t(const uint16_t* glu, const uint16_t* w2, const float* b2, const int32_t* order,
                          const float* route_w, uint16_t* out, int T, int H, int F, int K, hipStream_t s) {
    const bool one = T * K <= kDnWaves;  // at most one pair per wave
    if constexpr (MAXC <= 2) {
        if (H / 4 >= 2 * dec_cu_count()) {
            if (one) launch_down_k<HAS_BIAS, MAXC, 1, 4>(glu, w2, b2, order, route_w, out, T, H, F, K, s);
            else launch_down_k<HAS_BIAS, MAXC, 2, 4>(glu, w2, b2, order, route_w, out, T, H, F, K, s);
            return;
        }
    }
    if (one || MAXC > 4) launch_down_k<HAS_BIAS, MAXC, 1, 2>(glu, w2, b2, order, route_w, out, T, H, F, K, s);
    else launch_down_k<HAS_BIAS, MAXC, (MAXC <= 4 ? 2 : 1), 2>(glu, w2, b2, order, route_w, out, T, H, F, K, s);
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
    case C: launch_gateup_t<ACT, BIAS, C>(x, w1, b1, idx, glu, order, T, H, F, E, K, s); break;
#define CMOE_DEC_GU_ALL(ACT, BIAS) \
    switch (cg) { CMOE_DEC_GU(ACT, BIAS, 1) CMOE_DEC_GU(ACT, BIAS, 2) CMOE_DEC_GU(ACT, BIAS, 3) \
                  CMOE_DEC_GU(ACT, BIAS, 4) CMOE_DEC_GU(ACT, BIAS, 6) CMOE_DEC_GU(ACT, BIAS, 8) default: break; }
#define CMOE_DEC_DN(BIAS, C) \
    case C: launch_down_t<BIAS, C>(glu, w2, b2, order, route_w, out, T, H, F, K, s); break;
#define CMOE_DEC_DN_ALL(BIAS) \
    switch (cd) { CMOE_DEC_DN(BIAS, 1) CMOE_DEC_DN(BIAS, 2) CMOE_DEC_DN(BIAS, 3) CMOE_DEC_DN(BIAS, 4) \
                  CMOE_DEC_DN(BIAS, 6) CMOE_DEC_DN(BIAS, 8) default: break; }

bool decode_shape_supported(int H, int F) { return pick_maxc(H) > 0 && pick_maxc(F) > 0; }

hipError_t launch_decode(const uint16_t* x, const uint16_t* w1, const float* b1, const uint16_t* w2, const float* b2,
                         const int32_t* idx, const float* route_w, uint16_t* glu, int32_t* order, uint16_t* out,
                         int T, int H, int F, int E, int K, int act, hipStream_t s, hipEvent_t* ev) {
    // ev (optional): 3 events recorded before gate_up, after gate_up, after down.
    auto mark = [&](int i) { if (ev) (void)hipEventRecord(ev[i], s); };
    if (E > kDecMaxExperts) return hipErrorInvalidValue;
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

// ---- scratch of the allocation-free decode entry (cernels_moe_experts_decode_noalloc) --------------
// The workspace of the largest decode call the entry accepts: glu [kDecMaxPairs, 4096] bf16, then the
// expert-sorted pair order [kDecMaxPairs] int32, laid out as the decode workspace is (moe_capi.cpp,
// sections 256-byte aligned). Every GPU the library runs on holds its own copy until the process ends.
// The decode kernels write every byte they read from it, so nothing needs clearing between calls;
// calls that overlap on one GPU share it and race.
constexpr size_t kDecNoAllocBytes = (size_t)kDecMaxPairs * 4096 * 2 + (size_t)kDecMaxPairs * 4;
static_assert(kDecNoAllocBytes == CERNELS_MOE_DECODE_NOALLOC_SCRATCH_BYTES,
              "the public header states the scratch size");
static __device__ __align__(256) unsigned char scratch[kDecNoAllocBytes];

size_t decode_noalloc_bytes() { return kDecNoAllocBytes; }

// This GPU's address of `scratch` (in host code the name is only a stand-in, not a device address):
// looked up with hipGetSymbolAddress once per device, with that device current, and kept.
hipError_t decode_noalloc_scratch(void** ptr) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    int dev = 0;
    hipError_t st = hipGetDevice(&dev);
    if (st != hipSuccess) return st;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (addr[dev] == nullptr) {
        void* p = nullptr;
        st = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (st != hipSuccess) return st;
        if (p == nullptr) return hipErrorInvalidSymbol;
        addr[dev] = p;
    }
    *ptr = addr[dev];
    return hipSuccess;
}

}  // namespace cmoe
